"""Seeded inputs shared by the GPU parity tests: numpy data quantised by the CPU oracle, copied to
the GPU as the operands of the HIP kernels, so both sides see identical bytes."""

import sys

import numpy as np

F16, F32 = np.float16, np.float32


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def nf4_weight(rows, cols, seed, scale=0.02):
    """W ~ N(0, scale) fp16 [rows, cols] and its oracle NF4 double quant."""
    from oracle import nf4
    w = (np.random.default_rng(seed).standard_normal((rows, cols)) * scale).astype(F16)
    q = nf4.quantize(w)
    q["w"] = w
    q["deq"] = nf4.dequant(q["packed"], q["qabs"], q["scale2"], q["offset2"], q["code2"]).reshape(rows, cols)
    q["rows"], q["cols"] = rows, cols
    return q


def to_w4(q, device="cuda"):
    import torch
    from decentrik_prime_amd.w4linear import W4
    from decentrik_prime_amd.quant import nf4_table
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    return W4(t(q["packed"]), t(q["qabs"]), t(q["scale2"]), t(q["offset2"]), t(q["code2"]),
              nf4_table(device), q["rows"], q["cols"])


def cuda16(a, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=F16))).to(device)


def cuda(a, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    return t.detach().cpu().numpy()


def lora_inputs(m, k, n, r=16, seed=0, p=0.05):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(F16)
    a = (rng.uniform(-1, 1, (r, k)) / np.sqrt(k)).astype(F16)
    b = (rng.standard_normal((n, r)) * 0.02).astype(F16)
    mask = (rng.random((m, k)) >= p).astype(np.uint8)
    dy = (rng.standard_normal((m, n)) * 1e-2).astype(F16)
    return x, a, b, mask, dy


def assert_close(got, want, rtol, atol, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    lim = atol + rtol * np.abs(want)
    bad = ~(err <= lim)
    if bad.any():
        idx = np.unravel_index(np.argmax(err - lim), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside rtol {rtol} atol {atol}; "
                             f"worst at {idx}: got {got[idx]} want {want[idx]}")
