"""Write the golden fixtures of tests/golden/ from the CPU oracle (seeded, deterministic).

    python tests/golden/make_golden.py

Fixtures (all numpy .npz, no pickles):
  nf4_blocks.npz   three second-level blocks of random bytes/codes/scales (the shape of the
                   reference's emulator check, dev/test_emu.py:33-56) and their dequant
  nf4_vproj.npz    a v_proj-shaped weight [256, 1536] ~ N(0, 0.02), its NF4 double quant and dequant
  linear_small.npz a [128, 128] NF4 weight, LoRA r = 16, M = 64: forward and backward outputs
  mlp_small.npz    gated SiLU on [3, 2 x 1100] (the reference's odd width, dev/test_emu.py:307-322)
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import linear, mlp, nf4  # noqa: E402

F16, F32 = np.float16, np.float32


def nf4_blocks():
    rng = np.random.default_rng(0)
    n = 64 * 256 * 3
    nq = n // 64
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    qabs = rng.integers(0, 256, nq, dtype=np.uint8)
    code2 = np.sort(rng.uniform(-1, 1, 256)).astype(F32)
    scale2 = rng.uniform(0.001, 0.02, nq // 256).astype(F32)
    offset2 = np.repeat(rng.uniform(0.01, 0.03, 1).astype(F32), nq // 256)
    out = nf4.dequant(packed, qabs, scale2, offset2, code2)
    return dict(packed=packed, qabs=qabs, code2=code2, scale2=scale2, offset2=offset2,
                out=out.view(np.uint16))


def vproj_weight():
    return (np.random.default_rng(1).standard_normal((256, 1536)) * 0.02).astype(F16)


def nf4_vproj():
    w = vproj_weight()
    q = nf4.quantize(w)
    out = nf4.dequant(q["packed"], q["qabs"], q["scale2"], q["offset2"], q["code2"])
    # w itself is regenerated from default_rng(1) by the tests (see vproj_weight)
    return dict(packed=q["packed"], qabs=q["qabs"], scale2=q["scale2"],
                offset2=q["offset2"], code2=q["code2"], out=out.view(np.uint16))


def linear_small():
    rng = np.random.default_rng(2)
    m, k, n, r = 64, 128, 128, 16
    w = (rng.standard_normal((n, k)) * 0.02).astype(F16)
    q = nf4.quantize(w)
    wd = nf4.dequant(q["packed"], q["qabs"], q["scale2"], q["offset2"], q["code2"]).reshape(n, k)
    x = rng.standard_normal((m, k)).astype(F16)
    a = (rng.uniform(-1, 1, (r, k)) / np.sqrt(k)).astype(F16)
    b = (rng.standard_normal((n, r)) * 0.02).astype(F16)
    mask = (rng.random((m, k)) >= 0.05).astype(np.uint8)
    dy = (rng.standard_normal((m, n)) * 1e-2).astype(F16)
    ks = linear.keep_scale(0.05)
    y, z = linear.linear_fwd(x, wd, None, mask, ks, a, b, 2.0)
    g = linear.linear_bwd(dy, wd, z, x, mask, ks, a, b, 2.0)
    return dict(packed=q["packed"], qabs=q["qabs"], scale2=q["scale2"], offset2=q["offset2"],
                code2=q["code2"], x=x.view(np.uint16), a=a.view(np.uint16), b=b.view(np.uint16),
                mask=mask, dy=dy.view(np.uint16), y=y.view(np.uint16), z=z.view(np.uint16),
                dx=g["dx"], dA=g["dA"], dB=g["dB"], dZ=g["dZ"].view(np.uint16))


def mlp_small():
    rng = np.random.default_rng(3)
    n, inter = 3, 1100
    gu = (rng.standard_normal((n, 2 * inter)) * 2).astype(F16)
    dact = rng.standard_normal((n, inter)).astype(F16)
    return dict(gu=gu.view(np.uint16), dact=dact.view(np.uint16),
                act=mlp.gated_silu_fwd(gu).view(np.uint16),
                dgu=mlp.gated_silu_bwd(gu, dact).view(np.uint16))


FIXTURES = {"nf4_blocks": nf4_blocks, "nf4_vproj": nf4_vproj, "linear_small": linear_small,
            "mlp_small": mlp_small}


def main():
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
