"""GPU parity of the fp16-weight GEMM entry points (dk_h16_*, the GEMMs that read a weight already
dequantised to fp16, as the reference's GEMMs read its dequantised workspace,
solution/fast_qwen.py:694-756) and of the dequant-ahead schedule of the linear stack.

The fp16 weight is the GPU dequant of the NF4 weight (bit-exact with the oracle's, pinned by
test_gpu_nf4).  Where both entry points run the same kernel and tile plan (every shape here but
the long-K ones, which the fp16 path splits differently) the outputs must be bit-identical to the
dk_w4_* results; the long-K ones must agree to within fp32 summation-order differences (two fp16
ulps).  All are also checked against the oracle at rtol 1e-2 / atol 2e-2 (relative to the output
scale for the small-valued gradients)."""

import numpy as np
import pytest

from decentrik_prime_amd import _lib
from tests.helpers import assert_close, cuda, cuda16, host, log, lora_inputs, nf4_weight, to_w4

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-2, 2e-2
F16 = np.float16


def _scaled_close(got, want, what):
    s = float(np.abs(want).max()) or 1.0
    assert_close(np.asarray(got, np.float64) / s, np.asarray(want, np.float64) / s, RTOL, ATOL, what)


def _same(a, b, what):
    """Bit-identical tensors (fp16 / fp32 / uint8 alike)."""
    a, b = host(a), host(b)
    assert a.shape == b.shape and a.dtype == b.dtype, what
    if not np.array_equal(a.view(np.uint8), b.view(np.uint8)):
        bad = np.argwhere(a != b)
        raise AssertionError(f"{what}: {len(bad)} of {a.size} differ; first at {bad[0].tolist()}: "
                             f"{a[tuple(bad[0])]} vs {b[tuple(bad[0])]}")


def _abs_close(got, want, what):
    """rtol 1e-2 / atol 2e-2 on the values themselves (the forward outputs, of order 1)."""
    assert_close(np.asarray(got, np.float64), np.asarray(want, np.float64), RTOL, ATOL, what)


def _near(a, b, what):
    """Equal up to the rounding of a different fp32 summation order: two fp16 ulps of the value,
    plus one fp16 ulp at the tensor's scale for an fp16-rounded GEMM result that a bias or LoRA
    term then partly cancels."""
    a, b = host(a).astype(np.float64), host(b).astype(np.float64)
    scale = float(np.abs(b).max()) or 1.0
    tol = 2 * 2.0 ** -10 * np.abs(b) + 2.0 ** -11 * scale
    bad = np.abs(a - b) > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {a.size} differ beyond summation-order rounding"


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


@pytest.mark.parametrize("m", [2048, 200, 17])
def test_h16_fused_qkv(torch, m):
    """Fused QKV forward (two column-range LoRA terms, bias) and the dX GEMM with both masked LoRA
    terms, on the fp16 weight."""
    from decentrik_prime_amd import w4linear
    from oracle import linear
    log(f"h16 fused QKV forward + dX, M={m}")
    D, KV = 1536, 256
    q = nf4_weight(D + 2 * KV, D, seed=207)
    x, aq, bq, mq, _ = lora_inputs(m, D, D, seed=21)
    _, av, bv, mv, _ = lora_inputs(m, D, KV, seed=22)
    rng = np.random.default_rng(23)
    bias = (rng.standard_normal(D + 2 * KV) * 0.1).astype(F16)
    dqkv = (rng.standard_normal((m, D + 2 * KV)) * 1e-2).astype(F16)
    ks = linear.keep_scale(0.05)
    w = to_w4(q)
    w16 = w.dequantize()
    tzq = w4linear.lora_down(cuda16(x), cuda16(aq), cuda(mq), ks)
    tzv = w4linear.lora_down(cuda16(x), cuda16(av), cuda(mv), ks)
    terms = [(tzq, cuda16(bq), 0, D, 2.0), (tzv, cuda16(bv), D + KV, D + 2 * KV, 2.0)]
    y4 = w4linear.linear_forward_lora(cuda16(x), w, cuda16(bias), terms)
    y16 = w4linear.linear_forward_lora(cuda16(x), w, cuda16(bias), terms, w16=w16)
    torch.cuda.synchronize()
    _same(y16, y4, "qkv h16 vs w4")
    yq, _ = linear.linear_fwd(x, q["deq"][:D], bias[:D], mq, ks, aq, bq, 2.0)
    yk, _ = linear.linear_fwd(x, q["deq"][D:D + KV], bias[D:D + KV])
    yv, _ = linear.linear_fwd(x, q["deq"][D + KV:], bias[D + KV:], mv, ks, av, bv, 2.0)
    assert_close(host(y16), np.concatenate([yq, yk, yv], axis=1), RTOL, ATOL, "qkv vs oracle")
    g = cuda16(dqkv)
    dzq = (torch.randn(m, 16, device="cuda") * 1e-2).half()
    dzv = (torch.randn(m, 16, device="cuda") * 1e-2).half()
    bterms = [(dzq, cuda16(aq), cuda(mq), ks), (dzv, cuda16(av), cuda(mv), ks)]
    dx4 = w4linear.linear_backward_dx_lora(g, w, bterms)
    dx16 = w4linear.linear_backward_dx_lora(g, w, bterms, w16=w16)
    torch.cuda.synchronize()
    _same(dx16, dx4, "dX qkv h16 vs w4")
    mm = lambda a, b: linear.mm16(a, b).astype(np.float32)  # noqa: E731
    tq = np.where(mq != 0, mm(host(dzq), aq) * np.float32(ks), 0).astype(np.float32)
    tv = np.where(mv != 0, mm(host(dzv), av) * np.float32(ks), 0).astype(np.float32)
    _scaled_close(host(dx16), (mm(dqkv, q["deq"]) + tq) + tv, "dX qkv vs oracle")


def test_h16_o_projection(torch):
    """1536 x 1536 at M = 2048: 128 x 64 tiles with split-K in both directions; fp16 dX output
    and fp32 accumulation into an existing dX."""
    from decentrik_prime_amd import w4linear
    from oracle import linear
    log("h16 o projection forward + dX (split-K), M=2048")
    q = nf4_weight(1536, 1536, seed=208)
    rng = np.random.default_rng(24)
    x = rng.standard_normal((2048, 1536)).astype(F16)
    dy = (rng.standard_normal((2048, 1536)) * 1e-2).astype(F16)
    w = to_w4(q)
    w16 = w.dequantize()
    y4 = w4linear.linear_forward(cuda16(x), w)
    y16 = w4linear.linear_forward(cuda16(x), w, w16=w16)
    d4 = w4linear.linear_backward_dx(cuda16(dy), w, out_dtype=torch.float16)
    d16 = w4linear.linear_backward_dx(cuda16(dy), w, out_dtype=torch.float16, w16=w16)
    acc = torch.ones(2048, 1536, dtype=torch.float32, device="cuda")
    w4linear.linear_backward_dx(cuda16(dy), w, out=acc, accumulate=True, w16=w16)
    torch.cuda.synchronize()
    _same(y16, y4, "o forward h16 vs w4")
    _same(d16, d4, "o dX h16 vs w4")
    assert_close(host(y16), linear.mm16(x, q["deq"].T), RTOL, ATOL, "o forward vs oracle")
    ref = linear.mm16(dy, q["deq"])
    _scaled_close(host(d16), ref, "o dX vs oracle")
    _scaled_close(host(acc) - 1.0, ref.astype(np.float32), "o dX accumulate")


# M = 2300: 9 row tiles, so the down^T SwiGLU backward has 315 tiles (256 full + 59 leftover as
# 236 quarter workgroups, dispatched first: a count that is not a multiple of the 8 XCDs); M = 1:
# one token, every tile's rows but the first clamped
@pytest.mark.parametrize("m", [2048, 2300, 300, 1])
def test_h16_mlp(torch, m):
    """gate|up SwiGLU forward, down forward, down^T + SwiGLU backward and gate|up^T on fp16
    weights."""
    from decentrik_prime_amd import w4linear
    from oracle import linear, mlp
    log(f"h16 MLP forward + backward, M={m}")
    I = 8960
    qg = nf4_weight(2 * I, 1536, seed=204)
    qd = nf4_weight(1536, I, seed=205)
    wg, wd = to_w4(qg), to_w4(qd)
    g16, d16 = wg.dequantize(), wd.dequantize()
    x = np.random.default_rng(25).standard_normal((m, 1536)).astype(F16)
    act4, gu4 = w4linear.gateup_swiglu_forward(cuda16(x), wg)
    act16, gu16 = w4linear.gateup_swiglu_forward(cuda16(x), wg, w16=g16)
    torch.cuda.synchronize()
    _same(gu16, gu4, "gu h16 vs w4")
    _same(act16, act4, "act h16 vs w4")
    gu_ref, h_ref, _ = mlp.mlp_fwd(x, qg["deq"], qd["deq"])
    assert_close(host(gu16), gu_ref, RTOL, ATOL, "gu vs oracle")
    assert_close(host(act16), h_ref, RTOL, ATOL, "act vs oracle")
    y4 = w4linear.linear_forward(act16, wd)
    y16 = w4linear.linear_forward(act16, wd, w16=d16)
    torch.cuda.synchronize()
    _near(y16, y4, "down h16 vs w4")      # K = 8960: split differently
    assert_close(host(y16), linear.mm16(host(act16), qd["deq"].T), RTOL, ATOL, "down vs oracle")
    dh = (np.random.default_rng(26).standard_normal((m, 1536)) * 1e-2).astype(F16)
    gu_np = host(gu16)
    w4linear.down_swiglu_backward(cuda16(dh), wd, gu4)
    w4linear.down_swiglu_backward(cuda16(dh), wd, gu16, w16=d16)
    torch.cuda.synchronize()
    _same(gu16, gu4, "dgu h16 vs w4")
    dgu_ref, dx_ref = mlp.mlp_bwd(dh, gu_np, qg["deq"], qd["deq"])
    _scaled_close(host(gu16), dgu_ref, "dgu vs oracle")
    dx4 = w4linear.linear_backward_dx(gu4, wg, out_dtype=torch.float16)
    dx16 = w4linear.linear_backward_dx(gu16, wg, out_dtype=torch.float16, w16=g16)
    torch.cuda.synchronize()
    _near(dx16, dx4, "dX mlp h16 vs w4")  # K = 17920: split differently
    _scaled_close(host(dx16), dx_ref, "dX mlp vs oracle chain")


# M = 1900: the last row tile is partial while the fp16 SwiGLU GEMMs still run as persistent
# workgroups (8 row tiles), so the persistent walk's row guards are checked against the
# one-tile-per-workgroup NF4 tile kernel
@pytest.mark.parametrize("m", [2048, 1900, 1000])
def test_w4_tile_kernel_reads_nf4(torch, m):
    """Weights marked DK_W4_KERNEL_TILE: every NF4-reading GEMM whose shape the 256-tile plan
    takes runs on that kernel with its workgroups dequantising the W tiles into LDS (256 x 256
    tiles, the 128 x 128 quarters, split K; NT and NN; linear with LoRA terms and bias, the SwiGLU
    forward and backward), and must give the same bits as the fp16-weight form, which runs the
    same plan on the GPU-dequantised weight.  The gate|up forward and the down forward are also
    checked against the oracle directly (fp32 GEMMs of the oracle's dequantised weights)."""
    from decentrik_prime_amd import w4linear
    from oracle import linear
    log(f"W4 tile kernel vs fp16 form, M={m}")
    D, KV, I = 1536, 256, 8960
    rng = np.random.default_rng(41)
    w_qkv = to_w4(nf4_weight(D + 2 * KV, D, seed=211))
    w_o = to_w4(nf4_weight(D, D, seed=212))
    w_gu = to_w4(nf4_weight(2 * I, D, seed=213))
    w_d = to_w4(nf4_weight(D, I, seed=214))
    h = {k: w.dequantize() for k, w in (("qkv", w_qkv), ("o", w_o), ("gu", w_gu), ("d", w_d))}
    x, aq, bq, mq, _ = lora_inputs(m, D, D, seed=42)
    _, av, bv, mv, _ = lora_inputs(m, D, KV, seed=43)
    ks = linear.keep_scale(0.05)
    bias = cuda16((rng.standard_normal(D + 2 * KV) * 0.1).astype(F16))
    tx = cuda16(x)
    tzq = w4linear.lora_down(tx, cuda16(aq), cuda(mq), ks)
    tzv = w4linear.lora_down(tx, cuda16(av), cuda(mv), ks)
    fterms = [(tzq, cuda16(bq), 0, D, 2.0), (tzv, cuda16(bv), D + KV, D + 2 * KV, 2.0)]
    dqkv = cuda16((rng.standard_normal((m, D + 2 * KV)) * 1e-2).astype(F16))
    dzq = (torch.randn(m, 16, device="cuda") * 1e-2).half()
    dzv = (torch.randn(m, 16, device="cuda") * 1e-2).half()
    bterms = [(dzq, cuda16(aq), cuda(mq), ks), (dzv, cuda16(av), cuda(mv), ks)]
    dy_o = cuda16((rng.standard_normal((m, D)) * 1e-2).astype(F16))
    dh = cuda16((rng.standard_normal((m, D)) * 1e-2).astype(F16))

    def run(nf4):
        tile = _lib.DK_W4_KERNEL_TILE
        wq, wo, wg, wd = (w.with_kernel(tile) for w in (w_qkv, w_o, w_gu, w_d))
        pick = (lambda k: None) if nf4 else (lambda k: h[k])   # noqa: E731
        out = {}
        out["qkv"] = w4linear.linear_forward_lora(tx, wq, bias, fterms, w16=pick("qkv"))
        out["o"] = w4linear.linear_forward(tx, wo, w16=pick("o"))
        out["act"], gu = w4linear.gateup_swiglu_forward(tx, wg, w16=pick("gu"))
        out["gu"] = gu.clone()
        out["down"] = w4linear.linear_forward(out["act"], wd, w16=pick("d"))
        w4linear.down_swiglu_backward(dh, wd, gu, w16=pick("d"))
        out["dgu"] = gu
        out["dx_gu"] = w4linear.linear_backward_dx(gu, wg, out_dtype=torch.float16,
                                                   w16=pick("gu"))
        out["dx_o"] = w4linear.linear_backward_dx(dy_o, wo, w16=pick("o"))
        out["dx_qkv"] = w4linear.linear_backward_dx_lora(dqkv, wq, bterms, w16=pick("qkv"))
        return out

    want = run(False)
    got = run(True)
    torch.cuda.synchronize()
    for k in want:
        _same(got[k], want[k], f"{k}: W4 tile kernel vs fp16 form")
    # the oracle: gate|up forward (act and the saved [g | u]) and the down forward on the NF4
    # tile kernel's own act, at rtol 1e-2 / atol 2e-2
    from oracle import mlp
    gu_ref = linear.mm16(x, host(h["gu"]).reshape(2 * I, D).T)
    act_ref = mlp.gated_silu_fwd(gu_ref)
    _abs_close(host(got["act"]), act_ref, "act: W4 tile kernel vs oracle")
    _abs_close(host(got["gu"]), gu_ref, "[g | u]: W4 tile kernel vs oracle")
    down_ref = linear.mm16(host(got["act"]), host(h["d"]).reshape(D, I).T)
    _abs_close(host(got["down"]), down_ref, "down forward: W4 tile kernel vs oracle")


def test_w4_own_kernel_split_k(torch):
    """Weights marked DK_W4_KERNEL_STAGED: the split-K shapes at M = 2048 (down forward,
    K = 8960; gate|up dX, K = 17920), which AUTO gives to the 256-tile kernel, run on the NF4-form
    kernel's own split-K plan instead (its REDUCE launch).  Its summation order differs, so it is checked against the
    fp16 form at the split-K tolerance and against the oracle."""
    from decentrik_prime_amd import w4linear
    from oracle import linear
    m, D, I = 2048, 1536, 8960
    log(f"NF4-form kernel's own split-K, M={m}")
    qd, qg = nf4_weight(D, I, seed=231), nf4_weight(2 * I, D, seed=232)
    wd, wg = to_w4(qd), to_w4(qg)
    hd, hg = wd.dequantize(), wg.dequantize()
    rng = np.random.default_rng(233)
    act = (rng.standard_normal((m, I)) * 0.1).astype(np.float16)
    gu = (rng.standard_normal((m, 2 * I)) * 1e-2).astype(np.float16)
    tact, tgu = cuda16(act), cuda16(gu)
    want_y = w4linear.linear_forward(tact, wd, w16=hd)
    want_dx = w4linear.linear_backward_dx(tgu, wg, w16=hg)
    staged = _lib.DK_W4_KERNEL_STAGED
    got_y = w4linear.linear_forward(tact, wd.with_kernel(staged))
    got_dx = w4linear.linear_backward_dx(tgu, wg.with_kernel(staged))
    torch.cuda.synchronize()
    _near(got_y, want_y, "down forward: own split-K vs fp16 form")
    _near(got_dx, want_dx, "gate|up dX: own split-K vs fp16 form")
    _scaled_close(host(got_y), linear.mm16(act, qd["deq"].T), "down forward vs oracle")
    _scaled_close(host(got_dx), gu.astype(np.float32) @ qg["deq"].astype(np.float32),
                  "gate|up dX vs oracle")


def test_w4_without_workspace(torch):
    """A NULL workspace: the NF4 GEMMs that would split K (down forward, K = 8960) or dequantise W
    into the workspace first (q|k|v forward, o dX) run in one phase with the dequant in LDS.
    Checked against the fp16 form at summation-order tolerance and against the oracle."""
    from decentrik_prime_amd import _lib, w4linear
    from oracle import linear
    lib = _lib.lib()
    m, D, KV, I = 2048, 1536, 256, 8960
    log(f"NF4 GEMMs without a workspace, M={m}")
    qd, qq, qo = nf4_weight(D, I, seed=241), nf4_weight(D + 2 * KV, D, seed=242), nf4_weight(D, D, seed=243)
    wd, wq, wo = to_w4(qd), to_w4(qq), to_w4(qo)
    rng = np.random.default_rng(244)
    act = (rng.standard_normal((m, I)) * 0.1).astype(F16)
    x = rng.standard_normal((m, D)).astype(F16)
    dy = (rng.standard_normal((m, D)) * 1e-2).astype(F16)
    stream = _lib.stream_handle(torch.device("cuda"))

    def fwd(a, w):
        y = torch.empty(m, w.rows, dtype=torch.float16, device="cuda")
        assert lib.dk_w4_linear_fwd(_lib.ptr(a), a.stride(0), m, w.c_ref(), None, None, None, 0, 2.0,
                                    _lib.ptr(y), y.stride(0), None, 0, stream) == 0
        return y

    ta, tx, tdy = cuda16(act), cuda16(x), cuda16(dy)
    y_d, y_q = fwd(ta, wd), fwd(tx, wq)
    dx_o = torch.empty(m, D, dtype=torch.float32, device="cuda")
    assert lib.dk_w4_linear_bwd_dx(_lib.ptr(tdy), tdy.stride(0), m, wo.c_ref(), None, None, 0, None,
                                   1.0, _lib.ptr(dx_o), dx_o.stride(0), _lib.DK_OUT_F32, None, 0,
                                   stream) == 0
    torch.cuda.synchronize()
    _near(y_d, w4linear.linear_forward(ta, wd, w16=wd.dequantize()), "down: no workspace vs fp16 form")
    _near(y_q, w4linear.linear_forward(tx, wq, w16=wq.dequantize()), "qkv: no workspace vs fp16 form")
    _near(dx_o, w4linear.linear_backward_dx(tdy, wo, w16=wo.dequantize()), "o dX: no workspace vs fp16 form")
    assert_close(host(y_d), linear.mm16(act, qd["deq"].T), RTOL, ATOL, "down vs oracle")
    assert_close(host(y_q), linear.mm16(x, qq["deq"].T), RTOL, ATOL, "qkv vs oracle")
    _scaled_close(host(dx_o), linear.mm16(dy, qo["deq"]).astype(np.float32), "o dX vs oracle")


@pytest.mark.parametrize("m", [2048, 1900, 1000])
def test_split_k(torch, m):
    """The 256-tile kernel's split-K (fp32 partials in the workspace, summed in split order by a
    second launch that runs the epilogue) on a K = 8960 dX (NN, fp16, fp32 and fp32-accumulate
    outputs), and the down forward (NT, K = 8960), which splits K at M = 1000 (its 128 x 128
    quarters would fill less than half the CUs) and runs as quarters over the whole K at
    M = 2048 and 1900: against the oracle, and two calls bit-identical.  M = 1000 has ragged last
    rows and 10 splits per tile, M = 1900 ragged last rows (its last row quarters partial) and 5,
    M = 2048 has 5."""
    from decentrik_prime_amd import _lib, w4linear
    from oracle import linear
    lib = _lib.lib()
    I, D = 8960, 1536
    tiles = (m + 255) // 256 * (D // 256)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    splits = min(cus // tiles, I // 64 // 8)
    nt_quarters = (m + 127) // 128 * (D // 128)
    nt_split = nt_quarters * 2 < cus
    log(f"split-K, M={m}: {tiles} tiles x {splits} splits on {cus} CUs; NT split: {nt_split}")
    assert lib.dk_h16_workspace(m, D, I, _lib.DK_OP_LINEAR_FWD) == (
        tiles * splits * 256 * 256 * 4 if nt_split else 0)
    assert lib.dk_h16_workspace(m, I, D, _lib.DK_OP_LINEAR_BWD_DX) == tiles * splits * 256 * 256 * 4
    qd = nf4_weight(D, I, seed=301)      # down [1536, 8960]: NT, K = 8960
    qg = nf4_weight(I, D, seed=302)      # [8960, 1536]: dX = dy W, K = 8960
    wd, wg = to_w4(qd), to_w4(qg)
    d16, g16 = wd.dequantize(), wg.dequantize()
    rng = np.random.default_rng(303)
    x = (rng.standard_normal((m, I)) * 0.5).astype(F16)
    y1 = w4linear.linear_forward(cuda16(x), wd, w16=d16)
    y2 = w4linear.linear_forward(cuda16(x), wd, w16=d16)
    torch.cuda.synchronize()
    _same(y1, y2, "down forward, two calls")
    assert_close(host(y1), linear.mm16(x, qd["deq"].T), RTOL, ATOL, "down forward vs oracle")
    dy = (rng.standard_normal((m, I)) * 0.5).astype(F16)
    want = linear.mm16(dy, qg["deq"])
    dx16 = w4linear.linear_backward_dx(cuda16(dy), wg, out_dtype=torch.float16, w16=g16)
    dx32 = w4linear.linear_backward_dx(cuda16(dy), wg, out_dtype=torch.float32, w16=g16)
    base = torch.full((m, D), 0.25, dtype=torch.float32, device="cuda")
    acc = w4linear.linear_backward_dx(cuda16(dy), wg, out=base.clone(), accumulate=True, w16=g16)
    torch.cuda.synchronize()
    assert_close(host(dx16), want, RTOL, ATOL, "dX fp16 vs oracle")
    # fp32 output: fp32(fp16(dy W)), the same fp16 rounding as the fp16 output
    _same(dx32.half(), dx16, "dX fp32 output, rounded, vs fp16 output")
    _same(acc, dx32 + 0.25, "dX accumulate vs fp32 output + 0.25")


@pytest.mark.parametrize("m", [2048, 200])
def test_lora_multi_matches_single(torch, m):
    """The q and v adapters in shared launches (dk_lora_down_multi / dk_lora_grads_multi) give
    bit-identical results to one call per adapter, and those match the oracle."""
    from decentrik_prime_amd import w4linear
    from oracle import linear
    log(f"LoRA q+v shared launches vs one call each, M={m}")
    D, KV = 1536, 256
    x, aq, bq, mq, _ = lora_inputs(m, D, D, seed=31)
    _, av, bv, mv, _ = lora_inputs(m, D, KV, seed=32)
    ks = linear.keep_scale(0.05)
    dqkv = (np.random.default_rng(33).standard_normal((m, D + 2 * KV)) * 1e-2).astype(F16)
    tx, g = cuda16(x), cuda16(dqkv)
    t = {k: cuda16(v) for k, v in (("aq", aq), ("av", av), ("bq", bq), ("bv", bv))}
    tmq, tmv = cuda(mq), cuda(mv)
    zq1 = w4linear.lora_down(tx, t["aq"], tmq, ks)
    zv1 = w4linear.lora_down(tx, t["av"], tmv, ks)
    zq2, zv2 = w4linear.lora_down_multi(tx, [(t["aq"], tmq, ks), (t["av"], tmv, ks)])
    torch.cuda.synchronize()
    _same(zq2, zq1, "z_q")
    _same(zv2, zv1, "z_v")
    single = [w4linear.lora_grads(g[:, :D], zq1, tx, t["bq"], 2.0, tmq, ks),
              w4linear.lora_grads(g[:, D + KV:], zv1, tx, t["bv"], 2.0, tmv, ks)]
    multi = w4linear.lora_grads_multi(tx, [(g[:, :D], zq1, t["bq"], 2.0, tmq, ks),
                                           (g[:, D + KV:], zv1, t["bv"], 2.0, tmv, ks)])
    torch.cuda.synchronize()
    for term, (one, both) in zip("qv", zip(single, multi)):
        for nm, a, b in zip(("dA", "dB", "dz"), both, one):
            _same(a, b, f"{nm}_{term}")
    assert_close(host(zq1), linear.lora_down(x, mq, ks, aq), 2e-3, 2e-3, "z_q vs oracle")
    ref = linear.linear_bwd(dqkv[:, :D], np.zeros((D, D), F16), host(zq1), x, mq, ks, aq, bq, 2.0)
    for nm, got in zip(("dA", "dB", "dZ"), multi[0]):
        _scaled_close(host(got), ref[nm], f"{nm}_q vs oracle")


@pytest.mark.parametrize("m", [2048, 200])
def test_lora_down_with_dequant(torch, m):
    """dk_lora_down_multi_dequant: the q+v LoRA downs and a whole-layer dequant (or a block range
    of it) in one launch give z bit-identical to dk_lora_down_multi and fp16 weights
    bit-identical to dk_nf4_dequant, leaving the rest of the output untouched; masked terms,
    terms with their own inputs, and a masked beside an unmasked term (run as the separate
    calls)."""
    from decentrik_prime_amd import k_nf4, w4linear
    from decentrik_prime_amd.stack import NF4LinearStack
    from oracle import linear
    log(f"LoRA downs + layer dequant in one launch, M={m}")
    st = NF4LinearStack(1, 256, seed=7, device="cuda")
    pk, code2, nf4t = st.layers[0]["packed"], st.code2, st.nf4
    n_sb = pk.n_qblocks // 256
    whole = torch.empty(pk.numel, dtype=torch.float16, device="cuda")
    k_nf4.dequant_layer(pk, code2, nf4t, whole)
    D, KV = 1536, 256
    x, aq, _, mq, _ = lora_inputs(m, D, D, seed=51)
    _, av, _, mv, _ = lora_inputs(m, D, KV, seed=52)
    ks = linear.keep_scale(0.05)
    tx, taq, tav, tmq, tmv = cuda16(x), cuda16(aq), cuda16(av), cuda(mq), cuda(mv)
    xq = (torch.randn(m, D, device="cuda") * 0.5).half()
    xv = (torch.randn(m, D, device="cuda") * 0.5).half()
    cases = {"masked": (tx, [(taq, tmq, ks), (tav, tmv, ks)]),
             "own inputs": (None, [(taq, None, 1.0, xq), (tav, None, 1.0, xv)]),
             "mixed": (tx, [(taq, tmq, ks), (tav, None, 1.0)])}
    for name, (xin, terms) in cases.items():
        want = w4linear.lora_down_multi(xin, terms)
        for sb0, sb1 in ((0, n_sb), (3, n_sb - 5)):
            out = torch.full((pk.numel,), 7.0, dtype=torch.float16, device="cuda")
            side = k_nf4.side_dequant(pk, code2, nf4t, out, sb0, sb1, -1)
            got = w4linear.lora_down_multi(xin, terms, dequant=side)
            torch.cuda.synchronize()
            for t, (a, b) in enumerate(zip(got, want)):
                _same(a, b, f"{name} z[{t}], blocks [{sb0}, {sb1})")
            lo, hi = sb0 * 16384, sb1 * 16384
            _same(out[lo:hi], whole[lo:hi], f"{name} dequant, blocks [{sb0}, {sb1})")
            assert bool((out[:lo] == 7.0).all()) and bool((out[hi:] == 7.0).all()), \
                f"{name}: blocks outside [{sb0}, {sb1}) written"


@pytest.mark.parametrize("rank", [32, 64])
def test_lora_ranks_and_mixed_masks(torch, rank):
    """Ranks above the reference's 16 (the kernels take 16..64) and a masked term beside an
    unmasked one in the shared launches, ragged M: shared launches bit-identical to one call
    each, and the oracle's results (an unmasked term is the oracle's all-kept mask with scale 1)."""
    from decentrik_prime_amd import w4linear
    from oracle import linear
    m, D, KV = 300, 1536, 256
    log(f"LoRA rank {rank}, masked q + unmasked v, M={m}")
    x, aq, bq, mq, dyq = lora_inputs(m, D, D, r=rank, seed=41)
    _, av, bv, _, dyv = lora_inputs(m, D, KV, r=rank, seed=42)
    ks = linear.keep_scale(0.05)
    keep_all = np.ones_like(mq)
    tx = cuda16(x)
    t = {k: cuda16(v) for k, v in (("aq", aq), ("av", av), ("bq", bq), ("bv", bv),
                                   ("gq", dyq), ("gv", dyv))}
    tmq = cuda(mq)
    zq, zv = w4linear.lora_down_multi(tx, [(t["aq"], tmq, ks), (t["av"], None, 1.0)])
    zq1 = w4linear.lora_down(tx, t["aq"], tmq, ks)
    zv1 = w4linear.lora_down(tx, t["av"], None, 1.0)
    torch.cuda.synchronize()
    _same(zq, zq1, "z_q")
    _same(zv, zv1, "z_v")
    assert_close(host(zq), linear.lora_down(x, mq, ks, aq), 2e-3, 2e-3, "z_q vs oracle")
    assert_close(host(zv), linear.lora_down(x, keep_all, 1.0, av), 2e-3, 2e-3, "z_v vs oracle")
    multi = w4linear.lora_grads_multi(tx, [(t["gq"], zq, t["bq"], 2.0, tmq, ks),
                                           (t["gv"], zv, t["bv"], 2.0, None, 1.0)])
    single = [w4linear.lora_grads(t["gq"], zq, tx, t["bq"], 2.0, tmq, ks),
              w4linear.lora_grads(t["gv"], zv, tx, t["bv"], 2.0, None, 1.0)]
    torch.cuda.synchronize()
    for term, (both, one) in zip("qv", zip(multi, single)):
        for nm, a, b in zip(("dA", "dB", "dz"), both, one):
            _same(a, b, f"{nm}_{term}")
    for term, got, (dy, z, mk, kk, a, b, n) in zip(
            "qv", multi, ((dyq, zq, mq, ks, aq, bq, D), (dyv, zv, keep_all, 1.0, av, bv, KV))):
        ref = linear.linear_bwd(dy, np.zeros((n, D), F16), host(z), x, mk, kk, a, b, 2.0)
        for nm, g in zip(("dA", "dB", "dZ"), got):
            _scaled_close(host(g), ref[nm], f"{nm}_{term} vs oracle (rank {rank})")


def test_lora_per_term_inputs_and_zero_rows(torch):
    """Each term with its own input (the whole step's xq / xv, given with no mask) in the shared
    launches: bit-identical to one call per term on that input, and equal to the masked form on
    the common input wherever the dropout commutes with the rounding (the oracle's dropout of x is
    the input).  Zero rows: dA and dB come back as zeros (not left unwritten), z and dz empty."""
    from decentrik_prime_amd import w4linear
    from oracle import linear
    m, D, KV = 1024, 1536, 256
    log(f"LoRA per-term inputs, M={m}; zero rows")
    x, aq, bq, mq, dyq = lora_inputs(m, D, D, seed=51)
    _, av, bv, mv, dyv = lora_inputs(m, D, KV, seed=52)
    ks = linear.keep_scale(0.05)
    xq, xv = linear.dropout_input(x, mq, ks), linear.dropout_input(x, mv, ks)
    t = {k: cuda16(v) for k, v in (("xq", xq), ("xv", xv), ("aq", aq), ("av", av), ("bq", bq),
                                   ("bv", bv), ("gq", dyq), ("gv", dyv))}
    zq, zv = w4linear.lora_down_multi(None, [(t["aq"], None, 1.0, t["xq"]),
                                             (t["av"], None, 1.0, t["xv"])])
    zq1 = w4linear.lora_down(t["xq"], t["aq"])
    zv1 = w4linear.lora_down(t["xv"], t["av"])
    multi = w4linear.lora_grads_multi(None, [(t["gq"], zq, t["bq"], 2.0, None, 1.0, t["xq"]),
                                             (t["gv"], zv, t["bv"], 2.0, None, 1.0, t["xv"])])
    single = [w4linear.lora_grads(t["gq"], zq, t["xq"], t["bq"], 2.0),
              w4linear.lora_grads(t["gv"], zv, t["xv"], t["bv"], 2.0)]
    # the masked form on the common input gives the same Xd, so the same results
    tx = cuda16(x)
    masked = w4linear.lora_grads_multi(tx, [(t["gq"], zq, t["bq"], 2.0, cuda(mq), ks),
                                            (t["gv"], zv, t["bv"], 2.0, cuda(mv), ks)])
    torch.cuda.synchronize()
    _same(zq, zq1, "z_q")
    _same(zv, zv1, "z_v")
    for term, (both, one, msk) in zip("qv", zip(multi, single, masked)):
        for nm, a, b, c in zip(("dA", "dB", "dz"), both, one, msk):
            _same(a, b, f"{nm}_{term} per-term input vs one call")
            _same(a, c, f"{nm}_{term} per-term input vs masked common input")
    for term, got, (dy, z, a, b, n) in zip("qv", multi, ((dyq, zq, aq, bq, D), (dyv, zv, av, bv, KV))):
        ref = linear.linear_bwd(dy, np.zeros((n, D), F16), host(z), x, mq if term == "q" else mv,
                                ks, a, b, 2.0)
        for nm, g in zip(("dA", "dB", "dZ"), got):
            _scaled_close(host(g), ref[nm], f"{nm}_{term} vs oracle")
    # zero rows: dA, dB written as zeros over garbage, no input needed
    e16 = torch.empty(0, D, dtype=torch.float16, device="cuda")
    ez = torch.empty(0, 16, dtype=torch.float16, device="cuda")
    outs = [(torch.full((16, D), 7.0, device="cuda"), torch.full((n, 16), 7.0, device="cuda"),
             torch.empty(0, 16, dtype=torch.float16, device="cuda")) for n in (D, KV)]
    res = w4linear.lora_grads_multi(e16, [(torch.empty(0, D, dtype=torch.float16, device="cuda"), ez,
                                           t["bq"], 2.0, None, 1.0),
                                          (torch.empty(0, KV, dtype=torch.float16, device="cuda"), ez,
                                           t["bv"], 2.0, None, 1.0)], outs=outs)
    torch.cuda.synchronize()
    for da, db, dz in res:
        assert float(da.abs().max()) == 0.0 and float(db.abs().max()) == 0.0 and dz.numel() == 0


def test_h16_argument_checks(torch):
    from decentrik_prime_amd import w4linear
    log("h16 argument checks")
    q = nf4_weight(512, 256, seed=209)
    w = to_w4(q)
    x = torch.zeros(64, 256, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):   # wrong element count
        w4linear.linear_forward(x, w, w16=torch.zeros(512 * 128, dtype=torch.float16, device="cuda"))
    with pytest.raises(ValueError):   # wrong dtype
        w4linear.linear_forward(x, w, w16=torch.zeros(512, 256, dtype=torch.float32, device="cuda"))
    with pytest.raises(ValueError):   # not contiguous
        w4linear.linear_forward(x, w, w16=torch.zeros(256, 512, dtype=torch.float16,
                                                         device="cuda").t())


def test_stack_dequant_ahead_matches_nf4_reads(torch):
    """Three layers, M = 512, two steps: every weight dequantised one use ahead (per weight kind
    or the whole layer in one launch, in order on the compute stream or on a side stream, or
    carried by the GEMM launches, which at M = 512 mostly fall back to launches of their own),
    gives bit-identical outputs and LoRA gradients to the schedule that reads NF4 directly (same
    seed, so the same weights and inputs)."""
    from decentrik_prime_amd.stack import NF4LinearStack
    log("stack: dequant-ahead schedules vs NF4 reads, 3 layers, M=512, 2 steps")
    configs = (((), "main"), (NF4LinearStack.KINDS, "main"), (("gu", "d"), "side"),
               (NF4LinearStack.KINDS, "side"), ("layer", "main"), ("layer", "side"),
               ("carried", "main"))
    runs = {}
    for ahead, where in configs:
        st = NF4LinearStack(n_layers=3, m=512, seed=3, device="cuda", ahead=ahead, dq_stream=where)
        results = []
        for _ in range(2):
            st.step()
            torch.cuda.synchronize()
            results.append([t.clone() for t in (st.out["qkv"], st.out["o"], st.out["y"],
                                                 st.dx_qkv, st.dx_o, st.dx_mlp)]
                           + [g.clone() for gr in st.grads for g in gr]
                           + [gu.clone() for gu in st.gu])
        runs[(ahead, where)] = results
        del st
    names = (["qkv", "o", "y", "dx_qkv", "dx_o", "dx_mlp"]
             + [f"grad{i}.{j}" for i in range(3) for j in range(4)] + [f"dgu{i}" for i in range(3)])
    base = runs[configs[0]]
    for cfg in configs[1:]:
        for step in range(2):
            for name, a, b in zip(names, base[step], runs[cfg][step]):
                _same(b, a, f"{cfg} step {step} {name}")


def _layer_and_reference(torch, seed=11):
    """One repacked Qwen2.5-1.5B layer (random NF4 weights) and its whole-layer fp16 dequant."""
    from decentrik_prime_amd import k_nf4
    from decentrik_prime_amd.stack import NF4LinearStack
    st = NF4LinearStack(n_layers=1, m=2048, seed=seed, device="cuda", ahead="layer")
    pk = st.layers[0]["packed"]
    ref = torch.empty(pk.numel, dtype=torch.float16, device="cuda")
    k_nf4.dequant_layer(pk, st.code2, st.nf4, ref)
    return st, pk, ref


def test_carried_dequant_is_the_standalone_dequant(torch):
    """Each fp16-weight entry point carrying a share of a layer's dequant (automatic and explicit
    workgroup counts, full-grid and declined shapes): the GEMM result is bit-identical to the same
    call without the carried work, the carried blocks are bit-identical to dk_nf4_dequant of the
    layer, and every other element of the destination is untouched."""
    from decentrik_prime_amd import k_nf4, w4linear
    log("carried dequant on the four fp16-weight entry points, M=2048 and M=200")
    st, pk, ref = _layer_and_reference(torch)
    L, lo = st.layers[0], st.lora[0]
    for t in st.z[0].values():
        t.copy_((torch.randn(t.shape, device="cuda") * 0.1).half())
    n_sb = pk.n_qblocks // 256
    sentinel = torch.full((pk.numel,), -3.5, dtype=torch.float16, device="cuda")
    w16 = {k: ref[pk.segments[n][0]:pk.segments[n][0] + L[k].rows * L[k].cols]
           for k, n in (("qkv", "q_proj"), ("o", "o_proj"), ("gu", "gate_proj"), ("d", "down_proj"))}
    dev = "cuda"
    x = torch.randn(2048, 1536, device=dev).half()
    dyq = (torch.randn(2048, 2048, device=dev) * 1e-2).half()
    dyd = (torch.randn(2048, 1536, device=dev) * 1e-2).half()
    dz = [(torch.randn(2048, 16, device=dev) * 1e-2).half() for _ in range(2)]

    def calls(m, side):
        gu = torch.randn(m, 2 * 8960, device=dev).half()
        return {
            "qkv fwd": lambda: w4linear.linear_forward_lora(
                x[:m], L["qkv"], lo["bias"], st.qkv_terms(0) if m == 2048 else (), w16=w16["qkv"],
                side=side),
            "o dX": lambda: w4linear.linear_backward_dx(dyd[:m], L["o"], out_dtype=torch.float16,
                                                        w16=w16["o"], side=side),
            "qkv dX": lambda: w4linear.linear_backward_dx_lora(
                dyq[:m], L["qkv"], [(dz[0][:m], lo["Aq"], lo["mq"][:m], st.keep_scale),
                                    (dz[1][:m], lo["Av"], lo["mv"][:m], st.keep_scale)],
                w16=w16["qkv"], side=side),
            "gate|up fwd": lambda: w4linear.gateup_swiglu_forward(x[:m], L["gu"], w16=w16["gu"],
                                                                  side=side),
            "down bwd": lambda: w4linear.down_swiglu_backward(dyd[:m], L["d"], gu, w16=w16["d"],
                                                              side=side),
        }

    for m in (2048, 200):
        for (sb0, sb1, wgs) in ((0, n_sb, -1), (37, 1001, 5), (n_sb - 3, n_sb, 1)):
            for name in calls(m, None):
                torch.manual_seed(5)
                plain = calls(m, None)[name]()
                out = sentinel.clone()
                side = k_nf4.side_dequant(pk, st.code2, st.nf4, out, sb0, sb1, wgs)
                torch.manual_seed(5)
                carried = calls(m, side)[name]()
                torch.cuda.synchronize()
                what = f"{name} M={m} blocks [{sb0}, {sb1}) wgs {wgs}"
                for a, b in zip(plain if isinstance(plain, tuple) else (plain,),
                                carried if isinstance(carried, tuple) else (carried,)):
                    if a is not None:
                        _same(b, a, what + ": GEMM result")
                e0, e1 = sb0 * 16384, sb1 * 16384
                _same(out[e0:e1], ref[e0:e1], what + ": carried blocks")
                _same(out[:e0], sentinel[:e0], what + ": before the range")
                _same(out[e1:], sentinel[e1:], what + ": after the range")


@pytest.mark.parametrize("m,rank", [(2048, 16), (200, 16), (2048, 32)])
def test_lora_sums_carried_by_the_dx_gemm(torch, m, rank):
    """lora_dz_multi, then the q|k|v dX GEMM carrying the column sums (dk_lora_dz_multi +
    dk_h16_linear_bwd_dx_lora_sums), against lora_grads_multi and the dX GEMM without them: dA,
    dB, dz and dX bit-identical.  M = 2048 carries them on the 256-tile launch (also beside a
    carried dequant share, which stays bit-identical to dk_nf4_dequant); M = 200 (a shape that
    kernel declines) and rank 32 run them as a launch of their own after the GEMM."""
    from decentrik_prime_amd import k_nf4, w4linear
    log(f"LoRA column sums carried by the q|k|v dX GEMM, M={m}, rank {rank}")
    st, pk, ref = _layer_and_reference(torch)
    L = st.layers[0]
    D, KV = 1536, 256
    w16 = ref[pk.segments["q_proj"][0]:pk.segments["q_proj"][0] + L["qkv"].rows * L["qkv"].cols]
    x, aq, bq, mq, _ = lora_inputs(m, D, D, r=rank, seed=51)
    _, av, bv, mv, _ = lora_inputs(m, D, KV, r=rank, seed=52)
    ks = 1.0 / 0.95
    dqkv = cuda16((np.random.default_rng(53).standard_normal((m, D + 2 * KV)) * 1e-2).astype(F16))
    tx = cuda16(x)
    t = {k: cuda16(v) for k, v in (("aq", aq), ("av", av), ("bq", bq), ("bv", bv))}
    tmq, tmv = cuda(mq), cuda(mv)
    zq, zv = w4linear.lora_down_multi(tx, [(t["aq"], tmq, ks), (t["av"], tmv, ks)])
    terms = [(dqkv[:, :D], zq, t["bq"], 2.0, tmq, ks), (dqkv[:, D + KV:], zv, t["bv"], 2.0, tmv, ks)]
    want = w4linear.lora_grads_multi(tx, terms)

    def dx_terms(g):
        return [(g[0][2], t["aq"], tmq, ks), (g[1][2], t["av"], tmv, ks)]
    dx_want = w4linear.linear_backward_dx_lora(dqkv, L["qkv"], dx_terms(want), w16=w16)
    n_sb = pk.n_qblocks // 256
    for side_blocks in ((None, (0, n_sb // 4)) if m == 2048 and rank == 16 else (None,)):
        side, out = None, None
        if side_blocks is not None:
            out = torch.full((pk.numel,), -3.5, dtype=torch.float16, device="cuda")
            side = k_nf4.side_dequant(pk, st.code2, st.nf4, out, *side_blocks, -1)
        sums = w4linear.lora_dz_multi(tx, terms)
        got = sums.grads
        dx = w4linear.linear_backward_dx_lora(dqkv, L["qkv"], dx_terms(got), w16=w16, side=side,
                                              sums=sums)
        torch.cuda.synchronize()
        what = f"M={m} rank {rank}" + (" with a carried dequant" if side else "")
        for term, (a, b) in zip("qv", zip(got, want)):
            for nm, u, v in zip(("dA", "dB", "dz"), a, b):
                _same(u, v, f"{nm}_{term}, {what}")
        _same(dx, dx_want, f"dX, {what}")
        if side is not None:
            e0, e1 = side_blocks[0] * 16384, side_blocks[1] * 16384
            _same(out[e0:e1], ref[e0:e1], what + ": carried blocks")
            assert bool((out[e1:] == -3.5).all()), what + ": past the carried blocks"


def test_stack_carried_matches_layer_schedule(torch):
    """Two layers, M = 2048 (the shapes whose launches carry the dequant on idle CUs), two steps:
    the carried schedule gives bit-identical outputs and gradients to whole-layer dequant launches
    of their own."""
    from decentrik_prime_amd.stack import NF4LinearStack
    log("stack: carried dequant vs whole-layer launches, 2 layers, M=2048, 2 steps")
    runs = {}
    for ahead in ("layer", "carried"):
        st = NF4LinearStack(n_layers=2, m=2048, seed=4, device="cuda", ahead=ahead)
        results = []
        for _ in range(2):
            st.step()
            torch.cuda.synchronize()
            results.append([t.clone() for t in (st.out["qkv"], st.out["o"], st.out["y"],
                                                 st.dx_qkv, st.dx_o, st.dx_mlp)]
                           + [g.clone() for gr in st.grads for g in gr]
                           + [gu.clone() for gu in st.gu])
        runs[ahead] = results
        del st
    names = (["qkv", "o", "y", "dx_qkv", "dx_o", "dx_mlp"]
             + [f"grad{i}.{j}" for i in range(2) for j in range(4)] + [f"dgu{i}" for i in range(2)])
    for step in range(2):
        for name, a, b in zip(names, runs["layer"][step], runs["carried"][step]):
            _same(b, a, f"carried step {step} {name}")
