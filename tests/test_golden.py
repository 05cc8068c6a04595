"""The oracle reproduces the committed golden fixtures (tests/golden/make_golden.py)."""

import os

import numpy as np

from oracle import linear, mlp, nf4

GOLD = os.path.join(os.path.dirname(__file__), "golden")
F16 = np.float16


def load(name):
    return np.load(os.path.join(GOLD, name + ".npz"))


def h(a):
    return np.asarray(a).view(F16)


def test_nf4_blocks_fixture():
    g = load("nf4_blocks")
    out = nf4.dequant(g["packed"], g["qabs"], g["scale2"], g["offset2"], g["code2"])
    assert np.array_equal(out.view(np.uint16), g["out"])


def test_nf4_vproj_fixture():
    g = load("nf4_vproj")
    w = (np.random.default_rng(1).standard_normal((256, 1536)) * 0.02).astype(F16)
    q = nf4.quantize(w)
    for key in ("packed", "qabs", "scale2", "offset2", "code2"):
        assert np.array_equal(q[key], g[key]), key
    out = nf4.dequant(g["packed"], g["qabs"], g["scale2"], g["offset2"], g["code2"])
    assert np.array_equal(out.view(np.uint16), g["out"])


def test_linear_small_fixture():
    g = load("linear_small")
    wd = nf4.dequant(g["packed"], g["qabs"], g["scale2"], g["offset2"], g["code2"]).reshape(128, 128)
    ks = linear.keep_scale(0.05)
    y, z = linear.linear_fwd(h(g["x"]), wd, None, g["mask"], ks, h(g["a"]), h(g["b"]), 2.0)
    np.testing.assert_array_equal(z.view(np.uint16), g["z"])
    # fp32 CPU GEMM summation order can differ across thread counts: 1 fp16 ulp
    np.testing.assert_allclose(y.astype(np.float32), h(g["y"]).astype(np.float32), rtol=2e-3, atol=1e-4)
    gr = linear.linear_bwd(h(g["dy"]), wd, h(g["z"]), h(g["x"]), g["mask"], ks, h(g["a"]), h(g["b"]), 2.0)
    for key in ("dx", "dA", "dB"):
        np.testing.assert_allclose(gr[key], g[key], rtol=2e-3, atol=1e-6)


def test_mlp_small_fixture():
    g = load("mlp_small")
    assert np.array_equal(mlp.gated_silu_fwd(h(g["gu"])).view(np.uint16), g["act"])
    assert np.array_equal(mlp.gated_silu_bwd(h(g["gu"]), h(g["dact"])).view(np.uint16), g["dgu"])
