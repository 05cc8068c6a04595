"""CPU checks of the boundary: libdk.so loads, exports every entry point include/dk.h declares,
rejects bad arguments before any launch, and the Python mirror keeps the reference's rules."""

import ctypes
import os

import pytest
import torch

from decentrik_prime_amd import _lib, k_nf4, stack


def test_library_exports_every_declared_symbol():
    names = _lib.header_symbols()
    assert len(names) >= 14
    lib = _lib.lib()
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures and header disagree"


def test_built_for_gfx950():
    blob = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_argument_errors_come_back_before_launch():
    lib = _lib.lib()
    # null pointers / negative sizes -> DK_ERR_INVALID, without touching a device
    assert lib.dk_nf4_dequant(None, None, None, None, None, None, None, 4, None) == _lib.DK_ERR_INVALID
    assert lib.dk_nf4_dequant(None, None, None, None, None, None, None, -1, None) == _lib.DK_ERR_INVALID
    assert lib.dk_lora_down(None, None, 1.0, None, None, 8, 64, 16, None) == _lib.DK_ERR_INVALID
    w = _lib.NF4WeightC(1, 1, 1, 1, 1, 1, 100, 100)     # 10000 weights: not whole 16384 blocks
    assert lib.dk_w4_linear_fwd(ctypes.c_void_p(16), 100, 8, ctypes.byref(w), None, None, None, 0,
                                2.0, ctypes.c_void_p(16), 100, None, 0, None) == _lib.DK_ERR_INVALID
    assert lib.dk_w4_linear_workspace(2048, ctypes.byref(w), 0) == 0
    # the per-weight kernel choice: AUTO, TILE or STAGED only, refused before any launch
    for bad in (3, -1):
        wk = _lib.NF4WeightC(16, 16, 16, 16, 16, 16, 1536, 1536, bad)
        assert lib.dk_w4_linear_fwd(ctypes.c_void_p(16), 1536, 8, ctypes.byref(wk), None, None, None,
                                    0, 2.0, ctypes.c_void_p(16), 1536, None, 0,
                                    None) == _lib.DK_ERR_INVALID
        assert lib.dk_w4_workspace(2048, ctypes.byref(wk), _lib.DK_OP_LINEAR_FWD) == 0
    for good in (_lib.DK_W4_KERNEL_AUTO, _lib.DK_W4_KERNEL_TILE, _lib.DK_W4_KERNEL_STAGED):
        wk = _lib.NF4WeightC(16, 16, 16, 16, 16, 16, 1536, 1536, good)
        assert lib.dk_w4_workspace(2048, ctypes.byref(wk), _lib.DK_OP_LINEAR_FWD) == 1536 * 1536 * 2
    # workspace sizes (no device access): split-K partials, and the fp16 weight of the two-phase
    # path (from 512 rows on, outputs of 1536 columns or more)
    wq = _lib.NF4WeightC(16, 16, 16, 16, 16, 16, 1536, 1536)
    wgu = _lib.NF4WeightC(16, 16, 16, 16, 16, 16, 17920, 1536)
    assert lib.dk_w4_workspace(2048, ctypes.byref(wq), _lib.DK_OP_LINEAR_FWD) == 1536 * 1536 * 2
    assert lib.dk_w4_workspace(256, ctypes.byref(wq), _lib.DK_OP_LINEAR_FWD) == 48 * 3 * 128 * 64 * 4
    assert lib.dk_w4_workspace(2048, ctypes.byref(wgu), _lib.DK_OP_GATEUP_SWIGLU_FWD) == 17920 * 1536 * 2
    assert lib.dk_w4_workspace(256, ctypes.byref(wgu), _lib.DK_OP_GATEUP_SWIGLU_FWD) == 0
    assert lib.dk_w4_workspace(2048, ctypes.byref(wq), 7) == 0
    # misaligned packed pointer and fp16 output (both need 16 bytes)
    assert lib.dk_nf4_dequant(ctypes.c_void_p(2), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              ctypes.c_void_p(16), 4, None) == _lib.DK_ERR_ALIGN
    assert lib.dk_nf4_dequant(ctypes.c_void_p(4), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              ctypes.c_void_p(16), 4, None) == _lib.DK_ERR_ALIGN
    # fp16-weight GEMMs: split-K partials only (no fp16 copy of the weight to make)
    assert lib.dk_h16_workspace(256, 1536, 1536, _lib.DK_OP_LINEAR_FWD) == 48 * 3 * 128 * 64 * 4
    assert lib.dk_h16_workspace(2048, 2048, 1536, _lib.DK_OP_LINEAR_FWD) == 0
    assert lib.dk_h16_workspace(2048, 17920, 1536, _lib.DK_OP_GATEUP_SWIGLU_FWD) == 0
    assert lib.dk_h16_workspace(0, 1536, 1536, _lib.DK_OP_LINEAR_FWD) == 0
    p16 = ctypes.c_void_p(16)
    assert lib.dk_h16_linear_fwd_lora(p16, 1536, 8, None, 1536, 1536, None, None, 0, 0, p16, 1536,
                                      None, 0, None, None) == _lib.DK_ERR_INVALID     # no weight
    assert lib.dk_h16_linear_fwd_lora(p16, 1536, 8, ctypes.c_void_p(8), 1536, 1536, None, None, 0,
                                      0, p16, 1536, None, 0, None, None) == _lib.DK_ERR_ALIGN
    assert lib.dk_h16_linear_fwd_lora(p16, 1536, 8, p16, 1000, 1536, None, None, 0, 0, p16, 1536,
                                      None, 0, None, None) == _lib.DK_ERR_INVALID     # rows % 64
    assert lib.dk_h16_linear_bwd_dx_lora(p16, 1536, 8, p16, 1536, 1536, None, 0, 0, p16, 1536, 9,
                                         None, 0, None, None) == _lib.DK_ERR_INVALID  # output mode
    assert lib.dk_h16_gateup_swiglu_fwd(p16, 1536, 8, p16, 17920 + 64, 1536, p16, None, None, 0,
                                        None, None) == _lib.DK_ERR_INVALID            # rows % 128
    assert lib.dk_h16_down_swiglu_bwd(p16, 1536, 8, p16, 1536, 8960, None, None, 0,
                                      None, None) == _lib.DK_ERR_INVALID              # no gu
    assert lib.dk_h16_linear_fwd_lora(p16, 1536, 0, p16, 1536, 1536, None, None, 0, 0, p16, 1536,
                                      None, 0, None, None) == 0                       # zero rows
    # carried dequant: rejected before any launch when malformed
    good = dict(packed=16, qabs=16, scale2=16, offset2=16, code2=16, nf4=16, out=16, sb0=0, sb1=4,
                wgs=-1)
    for bad, err in ((dict(wgs=-2), _lib.DK_ERR_INVALID), (dict(wgs=1025), _lib.DK_ERR_INVALID),
                     (dict(sb0=5), _lib.DK_ERR_INVALID), (dict(sb0=-1), _lib.DK_ERR_INVALID),
                     (dict(packed=None), _lib.DK_ERR_INVALID), (dict(nf4=None), _lib.DK_ERR_INVALID),
                     (dict(out=8), _lib.DK_ERR_ALIGN), (dict(packed=4), _lib.DK_ERR_ALIGN)):
        side = _lib.SideDequantC(**{**good, **bad})
        for call in (
                lambda: lib.dk_h16_linear_fwd_lora(p16, 1536, 8, p16, 1536, 1536, None, None, 0, 0,
                                                   p16, 1536, None, 0, ctypes.byref(side), None),
                lambda: lib.dk_h16_linear_bwd_dx_lora(p16, 1536, 8, p16, 1536, 1536, None, 0, 0, p16,
                                                      1536, 0, None, 0, ctypes.byref(side), None),
                lambda: lib.dk_h16_gateup_swiglu_fwd(p16, 1536, 8, p16, 17920, 1536, p16, None,
                                                     None, 0, ctypes.byref(side), None),
                lambda: lib.dk_h16_down_swiglu_bwd(p16, 1536, 8, p16, 1536, 8960, p16, None, 0,
                                                   ctypes.byref(side), None)):
            assert call() == err, bad
    # the LoRA gradients need no workspace (one pass over the rows per column block)
    assert lib.dk_lora_grads_workspace(2048, 1536, 1536, 16) == 0
    n_outs = (ctypes.c_int64 * 2)(1536, 256)
    assert lib.dk_lora_grads_multi_workspace(2048, 1536, 16, n_outs, 2) == 0
    down = (_lib.LoraDownTermC * 3)()
    assert lib.dk_lora_down_multi(p16, 8, 64, 16, down, 3, None) == _lib.DK_ERR_INVALID  # 3 terms
    assert lib.dk_lora_down_multi(p16, 8, 64, 16, down, 1, None) == _lib.DK_ERR_INVALID  # no A / z
    down[0] = _lib.LoraDownTermC(None, 1.0, ctypes.c_void_p(8), p16)
    assert lib.dk_lora_down_multi(p16, 8, 64, 16, down, 1, None) == _lib.DK_ERR_ALIGN
    # a term's own input: required when the call has no x, and 16-byte aligned
    down[0] = _lib.LoraDownTermC(None, 1.0, p16, p16, None)
    assert lib.dk_lora_down_multi(None, 8, 64, 16, down, 1, None) == _lib.DK_ERR_INVALID
    down[0] = _lib.LoraDownTermC(None, 1.0, p16, p16, ctypes.c_void_p(8))
    assert lib.dk_lora_down_multi(None, 8, 64, 16, down, 1, None) == _lib.DK_ERR_ALIGN
    # no rows: zero-element tensors have null data pointers, and nothing is read or written
    down[0] = _lib.LoraDownTermC(None, 1.0, p16, None)
    assert lib.dk_lora_down_multi(None, 0, 64, 16, down, 1, None) == 0
    grads = (_lib.LoraGradsTermC * 1)()
    assert lib.dk_lora_grads_multi(p16, 8, 64, 16, grads, 1, None, 0, None) == _lib.DK_ERR_INVALID
    grads[0] = _lib.LoraGradsTermC(p16, 64, 64, p16, ctypes.c_void_p(8), 2.0, None, 1.0, p16, p16, p16)
    assert lib.dk_lora_grads_multi(p16, 8, 64, 16, grads, 1, None, 0, None) == _lib.DK_ERR_ALIGN
    grads[0] = _lib.LoraGradsTermC(p16, 32, 64, p16, p16, 2.0, None, 1.0, p16, p16, p16)   # lddy < n_out
    assert lib.dk_lora_grads_multi(p16, 8, 64, 16, grads, 1, None, 0, None) == _lib.DK_ERR_INVALID
    grads[0] = _lib.LoraGradsTermC(p16, 64, 64, p16, p16, 2.0, None, 1.0, p16, p16, p16, None)
    assert lib.dk_lora_grads_multi(None, 8, 64, 16, grads, 1, None, 0, None) == _lib.DK_ERR_INVALID
    grads[0] = _lib.LoraGradsTermC(None, 64, 64, None, p16, 2.0, None, 1.0, p16, p16, None, None)
    assert lib.dk_lora_grads_multi(None, 8, 64, 16, grads, 1, None, 0, None) == _lib.DK_ERR_INVALID
    assert b"misaligned" in lib.dk_error_string(_lib.DK_ERR_ALIGN)
    with pytest.raises(ValueError):
        _lib.check(_lib.DK_ERR_INVALID, "probe")


def test_norm_and_rope_argument_errors_come_back_before_launch():
    lib = _lib.lib()
    p16, p8, p4 = ctypes.c_void_p(16), ctypes.c_void_p(8), ctypes.c_void_p(4)
    # RMSNorm: d range and multiple of 4, required pointers, masks with the dropout outputs
    assert lib.dk_rms_fwd(p16, None, None, p16, p16, p16, None, None, None, None, 4, 1538, 1e-6, 1.0,
                          None) == _lib.DK_ERR_INVALID
    assert lib.dk_rms_fwd(p16, None, None, p16, p16, p16, None, None, None, None, 4, 8192, 1e-6, 1.0,
                          None) == _lib.DK_ERR_INVALID
    assert lib.dk_rms_fwd(None, None, None, p16, p16, p16, None, None, None, None, 4, 1536, 1e-6, 1.0,
                          None) == _lib.DK_ERR_INVALID
    assert lib.dk_rms_fwd(p16, None, None, p16, p16, p16, p16, p16, None, None, 4, 1536, 1e-6, 1.0,
                          None) == _lib.DK_ERR_INVALID                 # dropout without masks
    assert lib.dk_rms_fwd(p8, None, None, p16, p16, p16, None, None, None, None, 4, 1536, 1e-6, 1.0,
                          None) == _lib.DK_ERR_ALIGN
    assert lib.dk_rms_bwd(p16, 0, None, p16, None, p16, p16, None, p16, None, None, None, None, None, 4,
                          1536, 1.0, None) == _lib.DK_ERR_INVALID        # no gscale
    assert lib.dk_rms_bwd(p16, 0, p16, p16, None, p16, p16, None, p16, p16, None, None, p16, p16, 4, 1536,
                          1.0, None) == _lib.DK_ERR_INVALID              # lq without lv
    assert lib.dk_rms_bwd(p4, 0, p16, p16, None, p16, p16, None, p16, None, None, None, None, None, 4,
                          1536, 1.0, None) == _lib.DK_ERR_ALIGN          # dy16 needs 8 bytes
    assert lib.dk_rms_fwd(p16, None, None, p16, p16, p16, None, None, None, None, 0, 1536, 1e-6, 1.0,
                          None) == 0                                     # zero rows
    # QKV epilogue: head size, GQA partial count, tables aligned
    assert lib.dk_qkv_epilogue_fwd(p16, p16, p16, p16, p16, p16, 4, 2.0, 12, 2, 100,
                                   None) == _lib.DK_ERR_INVALID         # hd % 8
    assert lib.dk_qkv_epilogue_fwd(p16, p16, p16, p16, p8, p16, 4, 2.0, 12, 2, 128,
                                   None) == _lib.DK_ERR_ALIGN
    assert lib.dk_qkv_epilogue_bwd(p16, p16, p16, 1, p16, p16, p16, p16, 4, 12, 2, 128, 0,
                                   None) == _lib.DK_ERR_INVALID         # gin >= 1
    assert lib.dk_qkv_epilogue_bwd(p8, p16, p16, 1, p16, p16, p16, p16, 4, 12, 2, 128, 6,
                                   None) == _lib.DK_ERR_ALIGN           # fp32 grads: 16 bytes
    assert lib.dk_qkv_epilogue_bwd(p8, p8, p8, 0, p16, p16, p16, p16, 0, 12, 2, 128, 1, None) == 0
    # the QKV GEMM with the rotary epilogue: head size 128, whole heads within the output, tables
    # aligned, the fp16 weight present
    def fused(rope, m=4, w16=p16):
        return lib.dk_h16_linear_fwd_rope(p16, 1536, m, w16, 2048, 1536, None, None, 0, 0,
                                          None if rope is None else ctypes.byref(rope), p16, 2048,
                                          None, None)
    # attention: head size 128, nq a multiple of nkv, pointers and alignment; no blocks = no launch
    assert lib.dk_attn_fwd(p16, p16, 1, p16, 4, 100, 12, 2, 64, p16, p16, None) == _lib.DK_ERR_INVALID
    assert lib.dk_attn_fwd(p16, p16, 1, p16, 4, 100, 12, 5, 128, p16, p16, None) == _lib.DK_ERR_INVALID
    assert lib.dk_attn_fwd(p16, p16, 1, p16, 4, 100, 12, 2, 128, None, p16, None) == _lib.DK_ERR_INVALID
    assert lib.dk_attn_fwd(p8, p16, 1, p16, 4, 100, 12, 2, 128, p16, p16, None) == _lib.DK_ERR_ALIGN
    assert lib.dk_attn_fwd(p16, p16, 1, p16, 0, 100, 12, 2, 128, None, None, None) == 0
    assert lib.dk_attn_bwd(p16, p16, p16, p16, p16, 1, p16, 4, 100, 12, 2, 128, p16, p16, p16, None,
                           None) == _lib.DK_ERR_INVALID                  # no dv
    assert lib.dk_attn_bwd(p16, p16, p16, p8, p16, 1, p16, 4, 100, 12, 2, 128, p16, p16, p16, p16,
                           None) == _lib.DK_ERR_ALIGN                    # dout
    assert lib.dk_attn_bwd(p16, p16, p16, p16, p16, 1, p16, 4, 0, 12, 2, 128, None, None, None, None,
                           None) == 0                                    # no tokens
    # LM head row kernels: chunk width a multiple of 8, n_lab within the rows, hidden a multiple of 4
    assert lib.dk_head_chunk(p16, p16, p16, p16, 8, 4, 100, 0, 1.0, 1536, None) == _lib.DK_ERR_INVALID
    assert lib.dk_head_chunk(p16, p16, p16, p16, 8, 9, 128, 0, 1.0, 1536, None) == _lib.DK_ERR_INVALID
    assert lib.dk_head_chunk(p16, p16, p16, None, 8, 4, 128, 0, 1.0, 1536, None) == _lib.DK_ERR_INVALID
    assert lib.dk_head_chunk(p8, p16, p16, p16, 8, 4, 128, 0, 1.0, 1536, None) == _lib.DK_ERR_ALIGN
    assert lib.dk_head_chunk(p16, p16, p16, None, 0, 0, 128, 0, 1.0, 1536, None) == 0
    # the argmax (an fp32 in the state) is exact below 2^24 columns; one workgroup per row
    assert lib.dk_head_chunk(p16, p16, p16, p16, 8, 4, 128, (1 << 24) - 64, 1.0, 1536,
                             None) == _lib.DK_ERR_INVALID
    assert lib.dk_head_chunk(p16, p16, p16, p16, 1 << 31, 4, 128, 0, 1.0, 1536,
                             None) == _lib.DK_ERR_INVALID
    assert lib.dk_head_finalize(p16, p16, p16, p16, p16, p16, p16, 1 << 31, 4, 1.0, 1.0, 1536,
                                None) == _lib.DK_ERR_INVALID
    assert lib.dk_head_finalize(p16, p16, p16, p16, None, p16, p16, 8, 4, 1.0, 1.0, 1536,
                                None) == _lib.DK_ERR_INVALID            # targets without E_t rows
    assert lib.dk_head_finalize(p16, p16, p16, p16, p16, p16, p4, 8, 4, 1.0, 1.0, 1536,
                                None) == _lib.DK_ERR_ALIGN
    ok = _lib.RopeC(p16, p16, p16, 128, 1792)
    assert fused(None) == _lib.DK_ERR_INVALID
    assert fused(ok, w16=None) == _lib.DK_ERR_INVALID
    assert fused(_lib.RopeC(p16, p16, p16, 64, 1792)) == _lib.DK_ERR_INVALID
    assert fused(_lib.RopeC(p16, p16, p16, 128, 1700)) == _lib.DK_ERR_INVALID
    assert fused(_lib.RopeC(p16, p16, p16, 128, 2176)) == _lib.DK_ERR_INVALID   # beyond the output
    assert fused(_lib.RopeC(p16, p8, p16, 128, 1792)) == _lib.DK_ERR_ALIGN
    assert fused(ok, m=0) == 0


def test_norm_and_rope_mirrors_check_arguments():
    from decentrik_prime_amd import k_norm, k_rope
    x = torch.zeros(4, 1536)
    w = torch.zeros(1536)
    with pytest.raises(ValueError):
        k_norm.rms_forward(x, w, None, torch.zeros(4), 1e-6, xq=torch.zeros(4, 1536).half())
    with pytest.raises(ValueError):
        k_norm.rms_forward(x, w, None, torch.zeros(4), 1e-6)     # CPU tensors
    with pytest.raises(ValueError):
        k_norm.rms_backward(x.half(), torch.ones(1), x, w, torch.zeros(4), x, lq=x.half())
    with pytest.raises(ValueError):
        k_rope.qkv_epilogue_forward(torch.zeros(4, 2048).half(), torch.zeros(4, 1536).half(),
                                    torch.zeros(4, 256).half(), torch.zeros(4, dtype=torch.int32),
                                    torch.zeros(8, 128), torch.zeros(8, 128), 2.0, 12, 2, 128)
    assert k_norm.warmup_specs(1536) == [] and k_rope.warmup_specs(12, 2, 128, 6, None) == []


def test_zero_rows_is_a_no_op():
    lib = _lib.lib()
    assert lib.dk_gated_silu_fwd(ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 64, None) == 0
    assert lib.dk_nf4_dequant(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              ctypes.c_void_p(16), 0, None) == 0


class _Layer:
    def __init__(self, n_qblocks):
        self.n_qblocks = n_qblocks
        self.packed = torch.zeros(n_qblocks * 32, dtype=torch.uint8)
        self.qabs = torch.zeros(n_qblocks, dtype=torch.uint8)
        self.scale2 = torch.zeros(-(-n_qblocks // 256))
        self.offset2 = torch.zeros(-(-n_qblocks // 256))


def test_dequant_range_alignment_rules():
    layer = _Layer(3000)
    out = torch.empty(3000 * 64, dtype=torch.float16)
    code2 = torch.zeros(256)
    nf4 = torch.zeros(16)
    for q0, q1, dst in ((256, 3000, None), (0, 1500, None), (0, 1024, 64)):
        with pytest.raises(ValueError):
            k_nf4.dequant_range(layer, q0, q1, code2, nf4, out, dst)
    # aligned, but CPU tensors: rejected by the operator's device check, still a ValueError
    with pytest.raises(ValueError):
        k_nf4.dequant_range(layer, 1024, 3000, code2, nf4, out)


def test_section_layout_matches_reference_sizes():
    # one Qwen2.5-1.5B layer: 46,792,704 weights = 731,136 first-level blocks, 24,150,400 bytes
    n_q = sum(r * c for r, c in stack.SHAPES.values()) // 64
    assert n_q == 731136
    offs, nbytes = k_nf4.section_layout(n_q)
    assert nbytes == 24150400
    assert offs == (0, 23396352, 24127488, 24138944)
    assert all(o % 64 == 0 for o in offs)


def test_layer_flops():
    # per-GEMM list: forward q, k, v, o, gate|up, down; LoRA downs/ups; dX of each projection;
    # LoRA backward dA, dz, dB, dX-term for q and v
    M, D, I, KV, r = 2048, 1536, 8960, 256, 16
    g = lambda m, n, k: 2 * m * n * k  # noqa: E731
    fwd = g(M, D, D) + 2 * g(M, KV, D) + g(M, D, D) + g(M, 2 * I, D) + g(M, D, I)
    lora_f = 2 * g(M, r, D) + g(M, D, r) + g(M, KV, r)
    lora_b = (g(r, D, M) + g(M, r, D) + g(D, r, M) + g(M, D, r)
              + g(r, D, M) + g(M, r, KV) + g(KV, r, M) + g(M, D, r))
    assert stack.FLOP_PER_LAYER_M2048 == 2 * fwd + lora_f + lora_b == 384282132480
    assert abs(28 * stack.FLOP_PER_LAYER_M2048 / 1e12 - 10.760) < 1e-3


def test_package_has_no_oracle_dependency():
    pkg = os.path.dirname(_lib.__file__)
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                text = open(os.path.join(root, f)).read()
                assert "import oracle" not in text and "from oracle" not in text, f
