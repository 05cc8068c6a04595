"""dk_h16_linear_bwd_dx_lora_noalloc (no workspace argument, split-K partials in the library's own
device array) against dk_h16_linear_bwd_dx_lora with a workspace of dk_h16_workspace bytes, both
through the C ABI: bit-identical outputs on two calls in a row, the second on a smaller input (a
different split plan over the same array, with both masked LoRA terms), so a partial left by the
first call must not leak into the second."""

import ctypes

import numpy as np
import pytest

from tests.helpers import log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


def _case(torch, m, rows, cols, with_lora, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dy = (torch.randn(m, rows, device="cuda", generator=g) * 1e-2).half()
    w16 = (torch.randn(rows, cols, device="cuda", generator=g) * 0.02).half()
    terms = []
    if with_lora:
        for _ in range(2):
            dz = (torch.randn(m, 16, device="cuda", generator=g) * 1e-2).half()
            a = (torch.randn(16, cols, device="cuda", generator=g) * 0.02).half()
            mask = (torch.rand(m, cols, device="cuda", generator=g) >= 0.05).to(torch.uint8)
            terms.append((dz, a, mask))
    return dy, w16, terms


def _terms_c(terms, ks):
    from decentrik_prime_amd import _lib
    arr = (_lib.LoraTermC * 2)()
    for i, (dz, a, mask) in enumerate(terms):
        arr[i] = _lib.LoraTermC(dz.data_ptr(), a.data_ptr(), mask.data_ptr(), 0, 0, ks)
    return arr


def _with_workspace(torch, dy, w16, terms, out_mode, ks):
    from decentrik_prime_amd import _lib
    lib = _lib.lib()
    m, rows = dy.shape
    cols = w16.shape[1]
    nbytes = int(lib.dk_h16_workspace(m, rows, cols, _lib.DK_OP_LINEAR_BWD_DX))
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device="cuda")
    out = torch.empty(m, cols, dtype=torch.float32 if out_mode else torch.float16, device="cuda")
    rc = lib.dk_h16_linear_bwd_dx_lora(dy.data_ptr(), dy.stride(0), m, w16.data_ptr(), rows, cols,
                                       _terms_c(terms, ks), len(terms), 16 if terms else 0,
                                       out.data_ptr(), cols, out_mode, ws.data_ptr(), nbytes, None,
                                       _lib.stream_handle())
    _lib.check(rc, "dk_h16_linear_bwd_dx_lora")
    return out, nbytes


def _no_alloc(torch, dy, w16, terms, out_mode, ks):
    from decentrik_prime_amd import _lib
    lib = _lib.lib()
    m, rows = dy.shape
    cols = w16.shape[1]
    out = torch.empty(m, cols, dtype=torch.float32 if out_mode else torch.float16, device="cuda")
    rc = lib.dk_h16_linear_bwd_dx_lora_noalloc(dy.data_ptr(), dy.stride(0), m, w16.data_ptr(), rows,
                                               cols, _terms_c(terms, ks), len(terms),
                                               16 if terms else 0, out.data_ptr(), cols, out_mode,
                                               None, _lib.stream_handle())
    _lib.check(rc, "dk_h16_linear_bwd_dx_lora_noalloc")
    return out


def test_noalloc_dx_matches_workspace_form(torch):
    from decentrik_prime_amd import _lib
    ks = float(np.float32(1.0) / np.float32(0.95))
    # gate|up dX of config 4 (K = 17920, fp16 out), then a smaller input with both masked LoRA
    # terms (K = 8960, fp32 out): both split K, the second over fewer partial tiles
    for m, rows, cols, lora, mode in ((2048, 17920, 1536, False, _lib.DK_OUT_F16),
                                      (1024, 8960, 1536, True, _lib.DK_OUT_F32)):
        log(f"no-alloc dX: M={m} K={rows} N={cols} lora={lora}")
        dy, w16, terms = _case(torch, m, rows, cols, lora, seed=m + rows)
        want, nbytes = _with_workspace(torch, dy, w16, terms, mode, ks)
        got = _no_alloc(torch, dy, w16, terms, mode, ks)
        torch.cuda.synchronize()
        assert 0 < nbytes <= _lib.DK_NOALLOC_SCRATCH_BYTES, nbytes      # the split-K plan ran
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), f"M={m}: differs"
        assert bool(torch.isfinite(got.float()).all())


def test_noalloc_dx_under_graph_capture(torch):
    """The no-alloc entry point captured in a HIP graph (torch.cuda.graph) after one call outside
    capture: every replay, with eager work and synchronisations between them, gives the bits of
    the workspace form, and so does an eager call afterwards."""
    from decentrik_prime_amd import _lib
    lib = _lib.lib()
    ks = float(np.float32(1.0) / np.float32(0.95))
    m, rows, cols = 1024, 8960, 1536
    log(f"no-alloc dX under graph capture: M={m} K={rows} N={cols}")
    dy, w16, terms = _case(torch, m, rows, cols, True, seed=7)
    want, _ = _with_workspace(torch, dy, w16, terms, _lib.DK_OUT_F32, ks)
    _no_alloc(torch, dy, w16, terms, _lib.DK_OUT_F32, ks)     # outside capture: the set-up call
    torch.cuda.synchronize()
    out = torch.empty(m, cols, dtype=torch.float32, device="cuda")
    arr = _terms_c(terms, ks)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.dk_h16_linear_bwd_dx_lora_noalloc(dy.data_ptr(), dy.stride(0), m, w16.data_ptr(),
                                                   rows, cols, arr, len(terms), 16, out.data_ptr(),
                                                   cols, _lib.DK_OUT_F32, None,
                                                   _lib.stream_handle())
    _lib.check(rc, "dk_h16_linear_bwd_dx_lora_noalloc (captured)")
    for r in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.uint8), want.view(torch.uint8)), f"replay {r} differs"
        # eager work on the same array between replays (a smaller plan)
        small, _, _ = _case(torch, 512, rows, cols, False, seed=r)
        _no_alloc(torch, small, w16, [], _lib.DK_OUT_F16, ks)
        torch.cuda.synchronize()
    got = _no_alloc(torch, dy, w16, terms, _lib.DK_OUT_F32, ks)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), "eager call after replays"
