"""Fused NF4 QLoRA linear operators (forward, dX backward, LoRA gradients, gate|up SwiGLU).

These replace the reference's dequant-to-workspace + ``torch.mm``/``addmm`` call sites and the
LoRA lines around them (solution/fast_qwen.py:943-947, 1037, 1080-1112, 1310-1383;
solution/k_norm.py:49-53, 65-71; solution/k_rope.py:39-43, 54-58).  A GEMM either reads the NF4
sections and dequantises its W tiles on the fly (``dk_w4_*`` in libdk.so) or, given ``w16``,
reads an fp16 copy of the weight dequantised ahead (``dk_h16_*``, the reference's dequantised
workspace).  Every op runs on ``torch.cuda.current_stream()`` and allocates only its outputs and
scratch (split-K partials, LoRA partial sums) through torch.
"""

import ctypes
import threading

import torch

from . import _lib
from .quant import code2_on, nf4_table


class W4:
    """An NF4 weight [rows, cols] on the GPU: views of the four sections plus the two tables.

    ``kernel`` (``_lib.DK_W4_KERNEL_*``) is the GEMM kernel the ``dk_w4_*`` calls on this weight
    run: AUTO (the library's choice), TILE (the 256-tile kernel reading NF4 wherever its plan
    takes the shape) or STAGED (never that kernel).  It travels with every call (the weight
    struct's ``kernel`` field); ``with_kernel`` gives another view of the same sections."""

    def __init__(self, packed, qabs, scale2, offset2, code2, nf4, rows, cols,
                 kernel=_lib.DK_W4_KERNEL_AUTO):
        self.packed, self.qabs, self.scale2, self.offset2 = packed, qabs, scale2, offset2
        self.code2, self.nf4 = code2, nf4
        self.rows, self.cols = int(rows), int(cols)
        if kernel not in (_lib.DK_W4_KERNEL_AUTO, _lib.DK_W4_KERNEL_TILE, _lib.DK_W4_KERNEL_STAGED):
            raise ValueError(f"unknown W4 kernel choice {kernel}")
        self.kernel = int(kernel)
        n = self.rows * self.cols
        if n % 16384:
            raise ValueError("an NF4 weight must fill whole second-level blocks (16384 weights)")
        if (packed.numel() != n // 2 or qabs.numel() != n // 64 or scale2.numel() != n // 16384
                or offset2.numel() != n // 16384):
            raise ValueError("NF4 section sizes do not match the weight shape")
        self._c = _lib.NF4WeightC(packed.data_ptr(), qabs.data_ptr(), scale2.data_ptr(),
                                  offset2.data_ptr(), code2.data_ptr(), nf4.data_ptr(),
                                  self.rows, self.cols, self.kernel)

    def with_kernel(self, kernel):
        """The same weight (the same section tensors) with another ``kernel`` choice."""
        return W4(self.packed, self.qabs, self.scale2, self.offset2, self.code2, self.nf4,
                  self.rows, self.cols, kernel)

    @property
    def shape(self):
        return (self.rows, self.cols)

    @property
    def device(self):
        return self.packed.device

    def c_ref(self):
        import ctypes
        return ctypes.byref(self._c)

    @classmethod
    def from_sections(cls, packed, qabs, scale2, offset2, start, rows, cols, code2, nf4):
        n = rows * cols
        if start % 16384:
            raise ValueError("weight does not start on a second-level block")
        return cls(packed[start // 2:(start + n) // 2], qabs[start // 64:(start + n) // 64],
                   scale2[start // 16384:(start + n) // 16384],
                   offset2[start // 16384:(start + n) // 16384], code2, nf4, rows, cols)

    @classmethod
    def from_params(cls, param, nf4=None):
        """From a Params4bit-like weight (``.data`` packed, ``.quant_state`` nested NF4)."""
        qs = param.quant_state
        rows, cols = int(qs.shape[0]), int(qs.shape[1])
        dev = param.data.device
        n = rows * cols
        offset2 = qs.offset.float().reshape(1).expand(n // 16384).contiguous().to(dev)
        return cls(param.data.reshape(-1), qs.absmax.reshape(-1), qs.state2.absmax.reshape(-1).float(),
                   offset2, qs.state2.code.float().to(dev),
                   nf4 if nf4 is not None else nf4_table(dev), rows, cols)

    def dequantize(self, out=None):
        """fp16 [rows, cols] (the reference's workspace view of this weight)."""
        from .k_nf4 import dequant_tensors
        if out is None:
            out = torch.empty(self.rows, self.cols, dtype=torch.float16, device=self.device)
        dequant_tensors(self.packed, self.qabs, self.scale2, self.offset2,
                        self.rows * self.cols // 64, self.code2, self.nf4, out.view(-1))
        return out


_WS = {}
_WS_LOCK = threading.Lock()


def _workspace(w, m, op, device):
    """Scratch of a fused NF4 GEMM (split-K partials and the two-phase fp16 weight; None when the
    shape needs none): one buffer per (device, stream), grown on demand.  Kernels on one stream
    run in order, so they share it."""
    nbytes = int(_lib.lib().dk_w4_workspace(m, w.c_ref(), int(op)))
    if nbytes == 0:
        return None, 0
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    with _WS_LOCK:
        buf = _WS.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = _WS[key] = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return buf, nbytes


def _h16_workspace(m, rows, cols, op, device):
    """Split-K scratch of an fp16-weight GEMM (None when the shape needs none)."""
    nbytes = int(_lib.lib().dk_h16_workspace(m, rows, cols, int(op)))
    if nbytes == 0:
        return None, 0
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    with _WS_LOCK:
        buf = _WS.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = _WS[key] = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return buf, nbytes


def _check_w16(w16, w):
    """An fp16 copy of NF4 weight w ([rows, cols] or flat), contiguous, on its device."""
    if w16.dtype != torch.float16 or not w16.is_cuda or not w16.is_contiguous():
        raise ValueError("w16 must be a contiguous CUDA fp16 tensor")
    if w16.numel() != w.rows * w.cols:
        raise ValueError(f"w16 has {w16.numel()} elements, the weight {w.rows} x {w.cols}")


def _side(side):
    """Pointer argument for a carried dequant (k_nf4.side_dequant) or None."""
    if side is None:
        return None
    if not isinstance(side, _lib.SideDequantC):
        raise ValueError("side must come from k_nf4.side_dequant")
    return ctypes.byref(side)


def _check16(t, name, shape=None):
    if t.dtype != torch.float16 or not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA fp16 tensor, got {t.dtype} on {t.device}")
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be 2-D with unit column stride")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def _mask_ok(mask, shape):
    if mask is None:
        return None
    if mask.dtype == torch.bool:
        mask = mask.view(torch.uint8)
    if mask.dtype != torch.uint8 or tuple(mask.shape) != tuple(shape) or not mask.is_contiguous():
        raise ValueError(f"mask must be a contiguous uint8/bool tensor of shape {tuple(shape)}")
    return mask


def lora_down(x, lora_A, mask=None, keep_scale=1.0, out=None):
    """z = fp16(drop(x) A^T), drop(x) = fp16(mask ? x * keep_scale : 0).  x [M, K], A [r, K]."""
    _check16(x, "x")
    m, k = x.shape
    _check16(lora_A, "lora_A")
    r = lora_A.shape[0]
    if lora_A.shape[1] != k or not x.is_contiguous() or not lora_A.is_contiguous():
        raise ValueError("lora_down: x [M, K] and A [r, K] must be contiguous and agree on K")
    mask = _mask_ok(mask, (m, k))
    if out is None:
        out = torch.empty(m, r, dtype=torch.float16, device=x.device)
    rc = _lib.lib().dk_lora_down(_lib.ptr(x), _lib.ptr(mask), float(keep_scale), _lib.ptr(lora_A),
                                 _lib.ptr(out), m, k, r, _lib.stream_handle(x.device))
    _lib.check(rc, "dk_lora_down")
    return out


def lora_down_multi(x, terms, outs=None, dequant=None):
    """lora_down of one or two adapters in shared launches (the q and v adapters of the fused QKV
    projection): terms = [(lora_A [r, K], mask or None, keep_scale[, x_term]), ...].  A term's
    input is x, or its own x_term [M, K] (the reference's xq / xv: the fp32 norm output dropped out
    per adapter, solution/k_norm.py:49-53, given with mask None); x may be None when every term has
    one.  dequant: a k_nf4.side_dequant description whose blocks the same launch dequantises
    (dk_lora_down_multi_dequant; its wgs is not used), or None.  Returns [z, ...], each exactly as
    lora_down computes it."""
    if not 1 <= len(terms) <= 2:
        raise ValueError("lora_down_multi takes one or two terms")
    ins = [t[3] if len(t) > 3 and t[3] is not None else x for t in terms]
    if any(u is None for u in ins):
        raise ValueError("lora_down_multi: a term without its own input needs x")
    for u in ins:
        _check16(u, "x")
        if not u.is_contiguous() or u.shape != ins[0].shape:
            raise ValueError("lora_down_multi: the inputs must be contiguous [M, K] of one shape")
    m, k = ins[0].shape
    r = terms[0][0].shape[0]
    arr = (_lib.LoraDownTermC * len(terms))()
    keep, zs = [], []
    for t, term in enumerate(terms):
        a, mask, ks = term[:3]
        _check16(a, "lora_A")
        if tuple(a.shape) != (r, k) or not a.is_contiguous():
            raise ValueError("lora_down_multi: every lora_A must be a contiguous [r, K]")
        mask = _mask_ok(mask, (m, k))
        z = outs[t] if outs is not None else torch.empty(m, r, dtype=torch.float16, device=a.device)
        _check16(z, "z", (m, r))
        own = ins[t] if ins[t] is not x else None
        arr[t] = _lib.LoraDownTermC(_lib.ptr(mask), float(ks), _lib.ptr(a), _lib.ptr(z),
                                    _lib.ptr(own))
        keep.append((a, mask))
        zs.append(z)
    if dequant is not None:
        rc = _lib.lib().dk_lora_down_multi_dequant(_lib.ptr(x), m, k, r, arr, len(terms),
                                                   ctypes.byref(dequant),
                                                   _lib.stream_handle(ins[0].device))
        _lib.check(rc, "dk_lora_down_multi_dequant")
        return zs
    rc = _lib.lib().dk_lora_down_multi(_lib.ptr(x), m, k, r, arr, len(terms),
                                       _lib.stream_handle(ins[0].device))
    _lib.check(rc, "dk_lora_down_multi")
    return zs


def linear_forward(x, w, bias=None, z=None, lora_B=None, lora_scale=2.0, out=None, w16=None,
                   side=None):
    """y = fp16(fp32(fp16(x W^T + bias)) + s * fp32(fp16(z B^T)))  (LoRA part optional).
    x [M, in] fp16, w a W4 [out, in], z [M, r], lora_B [out, r]; w16, side as in
    linear_forward_lora."""
    if side is not None and w16 is None:
        raise ValueError("a carried dequant (side) needs the fp16-weight form (w16)")
    if w16 is not None:
        if (z is None) != (lora_B is None):
            raise ValueError("z and lora_B go together")
        terms = [(z, lora_B, 0, w.rows, lora_scale)] if z is not None else []
        return linear_forward_lora(x, w, bias, terms, out, w16=w16, side=side)
    _check16(x, "x")
    m = x.shape[0]
    if x.shape[1] != w.cols:
        raise ValueError(f"x has {x.shape[1]} features, weight expects {w.cols}")
    if bias is not None:
        _check16(bias.view(1, -1), "bias", (1, w.rows))
    if (z is None) != (lora_B is None):
        raise ValueError("z and lora_B go together")
    r = 0
    if z is not None:
        r = z.shape[1]
        _check16(z, "z", (m, r))
        _check16(lora_B, "lora_B", (w.rows, r))
        if not z.is_contiguous() or not lora_B.is_contiguous():
            raise ValueError("z and lora_B must be contiguous")
    if out is None:
        out = torch.empty(m, w.rows, dtype=torch.float16, device=x.device)
    _check16(out, "out", (m, w.rows))
    ws, nbytes = _workspace(w, m, _lib.DK_OP_LINEAR_FWD, x.device)
    rc = _lib.lib().dk_w4_linear_fwd(_lib.ptr(x), x.stride(0), m, w.c_ref(), _lib.ptr(bias),
                                     _lib.ptr(z), _lib.ptr(lora_B), r, float(lora_scale),
                                     _lib.ptr(out), out.stride(0), _lib.ptr(ws), nbytes,
                                     _lib.stream_handle(x.device))
    _lib.check(rc, "dk_w4_linear_fwd")
    return out


def _lora_terms(terms, m, backward, n_cols):
    """ctypes array of dk_lora_term from (left, right, mask, col_begin, col_end, scale) tuples."""
    if len(terms) > 2:
        raise ValueError("at most two LoRA terms")
    arr = (_lib.LoraTermC * max(1, len(terms)))()
    rank = 0
    keep = []
    for i, (left, right, mask, c0, c1, scale) in enumerate(terms):
        r = left.shape[1]
        if rank and r != rank:
            raise ValueError("LoRA terms must share the rank")
        rank = r
        _check16(left, "LoRA left factor", (m, r))
        if backward:
            _check16(right, "lora_A", (r, n_cols))
            mask = _mask_ok(mask, (m, n_cols))
        else:
            _check16(right, "lora_B", (c1 - c0, r))
            if mask is not None:
                raise ValueError("forward LoRA terms take no mask")
        if not left.is_contiguous() or not right.is_contiguous():
            raise ValueError("LoRA factors must be contiguous")
        keep += [left, right, mask]
        arr[i] = _lib.LoraTermC(left.data_ptr(), right.data_ptr(),
                                mask.data_ptr() if mask is not None else None, c0, c1, float(scale))
    return arr, len(terms), rank, keep


def linear_forward_lora(x, w, bias=None, terms=(), out=None, w16=None, side=None):
    """The fused linear forward with up to two LoRA terms on disjoint output-column ranges:
    terms = [(z [M, r], lora_B [c1 - c0, r], col_begin c0, col_end c1, scale s), ...].  The fused
    QKV projection passes the q term on columns [0, NQ*HD) and the v term on the last NKV*HD
    columns (solution/fast_qwen.py:943-949).  w16: the weight already dequantised to fp16 (the
    reference's workspace view), or None to read the NF4 sections.  side (w16 only): dequant
    work the launch carries, from k_nf4.side_dequant, or None."""
    if side is not None and w16 is None:
        raise ValueError("a carried dequant (side) needs the fp16-weight form (w16)")
    _check16(x, "x")
    m = x.shape[0]
    if x.shape[1] != w.cols:
        raise ValueError(f"x has {x.shape[1]} features, weight expects {w.cols}")
    if bias is not None:
        _check16(bias.view(1, -1), "bias", (1, w.rows))
    arr, n, rank, _keep = _lora_terms([(z, b, None, c0, c1, s) for z, b, c0, c1, s in terms], m,
                                      False, w.rows)
    if out is None:
        out = torch.empty(m, w.rows, dtype=torch.float16, device=x.device)
    _check16(out, "out", (m, w.rows))
    if w16 is not None:
        _check_w16(w16, w)
        ws, nbytes = _h16_workspace(m, w.rows, w.cols, _lib.DK_OP_LINEAR_FWD, x.device)
        rc = _lib.lib().dk_h16_linear_fwd_lora(_lib.ptr(x), x.stride(0), m, _lib.ptr(w16), w.rows,
                                               w.cols, _lib.ptr(bias), arr, n, rank, _lib.ptr(out),
                                               out.stride(0), _lib.ptr(ws), nbytes, _side(side),
                                               _lib.stream_handle(x.device))
        _lib.check(rc, "dk_h16_linear_fwd_lora")
        return out
    ws, nbytes = _workspace(w, m, _lib.DK_OP_LINEAR_FWD, x.device)
    rc = _lib.lib().dk_w4_linear_fwd_lora(_lib.ptr(x), x.stride(0), m, w.c_ref(), _lib.ptr(bias),
                                          arr, n, rank, _lib.ptr(out), out.stride(0), _lib.ptr(ws),
                                          nbytes, _lib.stream_handle(x.device))
    _lib.check(rc, "dk_w4_linear_fwd_lora")
    return out


def linear_forward_rope(x, w, bias, terms, pos, cos, sin, rope_cols, out=None, w16=None,
                        side=None, hd=128):
    """linear_forward_lora of the fused QKV projection with the QKV epilogue's rotary embedding
    (solution/k_rope.py:23-61) folded into the GEMM epilogue: output columns [0, rope_cols) (the q
    and k heads, head size hd = 128) are rotated by the positions `pos` (int32 [M]) with the fp32
    tables cos/sin [positions, hd] before the single fp16 rounding, as the reference's epilogue
    kernel rotates q16 + s lq16.  Needs the fp16 weight (w16) and a shape the 256 x 256-tile
    kernel takes; side as in linear_forward_lora."""
    if w16 is None:
        raise ValueError("the rotary GEMM reads the fp16 weight (w16)")
    _check16(x, "x")
    m = x.shape[0]
    if x.shape[1] != w.cols:
        raise ValueError(f"x has {x.shape[1]} features, weight expects {w.cols}")
    if bias is not None:
        _check16(bias.view(1, -1), "bias", (1, w.rows))
    if pos.dtype != torch.int32 or not pos.is_cuda or tuple(pos.shape) != (m,):
        raise ValueError("pos must be a CUDA int32 [M] tensor")
    for t, nm in ((cos, "cos"), (sin, "sin")):
        if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous() or t.dim() != 2 \
                or t.shape[1] != hd:
            raise ValueError(f"{nm} must be a contiguous CUDA fp32 [positions, {hd}] table")
    arr, n, rank, _keep = _lora_terms([(z, b, None, c0, c1, s) for z, b, c0, c1, s in terms], m,
                                      False, w.rows)
    if out is None:
        out = torch.empty(m, w.rows, dtype=torch.float16, device=x.device)
    _check16(out, "out", (m, w.rows))
    _check_w16(w16, w)
    rope = _lib.RopeC(_lib.ptr(pos), _lib.ptr(cos), _lib.ptr(sin), int(hd), int(rope_cols))
    rc = _lib.lib().dk_h16_linear_fwd_rope(_lib.ptr(x), x.stride(0), m, _lib.ptr(w16), w.rows,
                                           w.cols, _lib.ptr(bias), arr, n, rank, ctypes.byref(rope),
                                           _lib.ptr(out), out.stride(0), _side(side),
                                           _lib.stream_handle(x.device))
    _lib.check(rc, "dk_h16_linear_fwd_rope")
    return out


def _dx_out(out, m, w, out_dtype, accumulate, device):
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs an output tensor")
        out = torch.empty(m, w.cols, dtype=out_dtype, device=device)
    if out.dtype == torch.float16:
        mode = _lib.DK_OUT_F16
        if accumulate:
            raise ValueError("accumulation is into fp32 only")
    elif out.dtype == torch.float32:
        mode = _lib.DK_OUT_F32_ACCUM if accumulate else _lib.DK_OUT_F32
    else:
        raise ValueError("dX is fp16 or fp32")
    if tuple(out.shape) != (m, w.cols) or out.stride(1) != 1:
        raise ValueError("dX output has the wrong shape or layout")
    return out, mode


def linear_backward_dx_lora(dy, w, terms=(), out=None, out_dtype=torch.float32, accumulate=False,
                            w16=None, side=None, sums=None):
    """dX = fp32(fp16(dy W)) + sum over terms of (mask ? fp32(fp16(dz A)) * keep_scale : 0),
    terms = [(dz [M, r], lora_A [r, in], mask [M, in] or None, keep_scale), ...] added in order
    (the QKV backward: dy1 = mm(dqkv, W_qkv) plus the lq and lv terms of rms_backward,
    solution/fast_qwen.py:1364, 1376-1380).  w16, side as in linear_forward_lora; sums (w16 form
    only) the LoraSums of lora_dz_multi, whose dA and dB this launch then computes as well."""
    if (side is not None or sums is not None) and w16 is None:
        raise ValueError("carried work (side, sums) needs the fp16-weight form (w16)")
    _check16(dy, "dy")
    m = dy.shape[0]
    if dy.shape[1] != w.rows:
        raise ValueError(f"dy has {dy.shape[1]} columns, weight has {w.rows} rows")
    arr, n, rank, _keep = _lora_terms([(dz, a, mk, 0, 0, ks) for dz, a, mk, ks in terms], m,
                                      True, w.cols)
    out, mode = _dx_out(out, m, w, out_dtype, accumulate, dy.device)
    if w16 is not None:
        _check_w16(w16, w)
        ws, nbytes = _h16_workspace(m, w.rows, w.cols, _lib.DK_OP_LINEAR_BWD_DX, dy.device)
        if sums is not None:
            rc = _lib.lib().dk_h16_linear_bwd_dx_lora_sums(
                _lib.ptr(dy), dy.stride(0), m, _lib.ptr(w16), w.rows, w.cols, arr, n, rank,
                _lib.ptr(out), out.stride(0), mode, _lib.ptr(ws), nbytes, _side(side),
                ctypes.byref(sums.c), _lib.stream_handle(dy.device))
            _lib.check(rc, "dk_h16_linear_bwd_dx_lora_sums")
            return out
        rc = _lib.lib().dk_h16_linear_bwd_dx_lora(_lib.ptr(dy), dy.stride(0), m, _lib.ptr(w16),
                                                  w.rows, w.cols, arr, n, rank, _lib.ptr(out),
                                                  out.stride(0), mode, _lib.ptr(ws), nbytes,
                                                  _side(side), _lib.stream_handle(dy.device))
        _lib.check(rc, "dk_h16_linear_bwd_dx_lora")
        return out
    ws, nbytes = _workspace(w, m, _lib.DK_OP_LINEAR_BWD_DX, dy.device)
    rc = _lib.lib().dk_w4_linear_bwd_dx_lora(_lib.ptr(dy), dy.stride(0), m, w.c_ref(), arr, n, rank,
                                             _lib.ptr(out), out.stride(0), mode, _lib.ptr(ws),
                                             nbytes, _lib.stream_handle(dy.device))
    _lib.check(rc, "dk_w4_linear_bwd_dx_lora")
    return out


def linear_backward_dx(dy, w, dz=None, lora_A=None, mask=None, keep_scale=1.0, out=None,
                       out_dtype=torch.float32, accumulate=False, w16=None, side=None):
    """dX = fp32(fp16(dy W)) + (mask ? fp32(fp16(dz A)) * keep_scale : 0).
    dy [M, out] fp16, w a W4 [out, in], dz [M, r], lora_A [r, in], mask [M, in].
    out_dtype float16 rounds dX to fp16; accumulate=True adds into an fp32 `out`; w16 as in
    linear_forward_lora."""
    if side is not None and w16 is None:
        raise ValueError("a carried dequant (side) needs the fp16-weight form (w16)")
    if w16 is not None:
        if (dz is None) != (lora_A is None):
            raise ValueError("dz and lora_A go together")
        terms = [(dz, lora_A, mask, keep_scale)] if dz is not None else []
        return linear_backward_dx_lora(dy, w, terms, out, out_dtype, accumulate, w16=w16,
                                       side=side)
    _check16(dy, "dy")
    m = dy.shape[0]
    if dy.shape[1] != w.rows:
        raise ValueError(f"dy has {dy.shape[1]} columns, weight has {w.rows} rows")
    if (dz is None) != (lora_A is None):
        raise ValueError("dz and lora_A go together")
    r = 0
    if dz is not None:
        r = dz.shape[1]
        _check16(dz, "dz", (m, r))
        _check16(lora_A, "lora_A", (r, w.cols))
        if not dz.is_contiguous() or not lora_A.is_contiguous():
            raise ValueError("dz and lora_A must be contiguous")
    mask = _mask_ok(mask, (m, w.cols))
    out, mode = _dx_out(out, m, w, out_dtype, accumulate, dy.device)
    ws, nbytes = _workspace(w, m, _lib.DK_OP_LINEAR_BWD_DX, dy.device)
    rc = _lib.lib().dk_w4_linear_bwd_dx(_lib.ptr(dy), dy.stride(0), m, w.c_ref(), _lib.ptr(dz),
                                        _lib.ptr(lora_A), r, _lib.ptr(mask), float(keep_scale),
                                        _lib.ptr(out), out.stride(0), mode, _lib.ptr(ws), nbytes,
                                        _lib.stream_handle(dy.device))
    _lib.check(rc, "dk_w4_linear_bwd_dx")
    return out


def lora_grads(dy, z, x, lora_B, lora_scale=2.0, mask=None, keep_scale=1.0):
    """(dA fp32 [r, in], dB fp32 [out, r], dz fp16 [M, r]) with
    dB = fp32(fp16(dy^T z)) s, dz = fp16(fp16(dy B) s), dA = fp32(fp16(dz^T drop(x))).
    dy may be a column slice (row stride > out), like the reference's gq = qkv[:, :NQ*HD]."""
    _check16(dy, "dy")
    for t, nm in ((z, "z"), (x, "x"), (lora_B, "lora_B")):
        _check16(t, nm)
        if not t.is_contiguous():
            raise ValueError(f"{nm} must be contiguous")
    m, n_out = dy.shape
    r = z.shape[1]
    k = x.shape[1]
    if z.shape[0] != m or x.shape[0] != m or tuple(lora_B.shape) != (n_out, r):
        raise ValueError("lora_grads: inconsistent shapes")
    mask = _mask_ok(mask, (m, k))
    dev = dy.device
    da = torch.empty(r, k, dtype=torch.float32, device=dev)
    db = torch.empty(n_out, r, dtype=torch.float32, device=dev)
    dz = torch.empty(m, r, dtype=torch.float16, device=dev)
    rc = _lib.lib().dk_lora_grads(_lib.ptr(dy), dy.stride(0), _lib.ptr(z), _lib.ptr(x),
                                  _lib.ptr(mask), float(keep_scale), _lib.ptr(lora_B),
                                  float(lora_scale), m, n_out, k, r, _lib.ptr(da), _lib.ptr(db),
                                  _lib.ptr(dz), None, 0, _lib.stream_handle(dev))
    _lib.check(rc, "dk_lora_grads")
    return da, db, dz


def _lora_grads_args(x, terms, outs):
    """Checked arguments of lora_grads_multi and lora_dz_multi: (ctypes term array, m, k, rank,
    device, tensors to keep alive, [(dA, dB, dz), ...])."""
    if not 1 <= len(terms) <= 2:
        raise ValueError("lora_grads_multi takes one or two terms")
    ins = [t[6] if len(t) > 6 and t[6] is not None else x for t in terms]
    if any(u is None for u in ins):
        raise ValueError("lora_grads_multi: a term without its own input needs x")
    for u in ins:
        _check16(u, "x")
        if not u.is_contiguous() or u.shape != ins[0].shape:
            raise ValueError("lora_grads_multi: the inputs must be contiguous [M, K] of one shape")
    m, k = ins[0].shape
    r = terms[0][1].shape[1]
    dev = ins[0].device
    arr = (_lib.LoraGradsTermC * len(terms))()
    keep, res = [x], []
    for t, term in enumerate(terms):
        dy, z, lora_B, s, mask, ks = term[:6]
        _check16(dy, "dy")
        for u, nm in ((z, "z"), (lora_B, "lora_B")):
            _check16(u, nm)
            if not u.is_contiguous():
                raise ValueError(f"{nm} must be contiguous")
        n_out = dy.shape[1]
        if dy.shape[0] != m or tuple(z.shape) != (m, r) or tuple(lora_B.shape) != (n_out, r):
            raise ValueError("lora_grads_multi: inconsistent shapes")
        mask = _mask_ok(mask, (m, k))
        if outs is not None:
            da, db, dz = outs[t]
            for u, shp, dt, nm in ((da, (r, k), torch.float32, "dA"), (db, (n_out, r), torch.float32, "dB"),
                                   (dz, (m, r), torch.float16, "dz")):
                if u.dtype != dt or tuple(u.shape) != shp or not u.is_contiguous():
                    raise ValueError(f"lora_grads_multi: {nm} must be a contiguous {dt} {shp}")
        else:
            da = torch.empty(r, k, dtype=torch.float32, device=dev)
            db = torch.empty(n_out, r, dtype=torch.float32, device=dev)
            dz = torch.empty(m, r, dtype=torch.float16, device=dev)
        own = ins[t] if ins[t] is not x else None
        arr[t] = _lib.LoraGradsTermC(_lib.ptr(dy), dy.stride(0), n_out, _lib.ptr(z),
                                     _lib.ptr(lora_B), float(s), _lib.ptr(mask), float(ks),
                                     _lib.ptr(da), _lib.ptr(db), _lib.ptr(dz), _lib.ptr(own))
        keep += [dy, z, lora_B, mask, own, da, db, dz]
        res.append((da, db, dz))
    return arr, m, k, r, dev, keep, res


def lora_grads_multi(x, terms, outs=None):
    """lora_grads of one or two adapters in shared launches: terms =
    [(dy, z, lora_B, lora_scale, mask or None, keep_scale[, x_term]), ...], x_term the term's own
    input (the reference's xq / xv, given with mask None) in place of x, which may then be None.
    outs: [(dA, dB, dz), ...] to write into, or None to allocate.  Returns [(dA, dB, dz), ...],
    each exactly as lora_grads computes it."""
    arr, m, k, r, dev, _keep, res = _lora_grads_args(x, terms, outs)
    rc = _lib.lib().dk_lora_grads_multi(_lib.ptr(x), m, k, r, arr, len(terms), None, 0,
                                        _lib.stream_handle(dev))
    _lib.check(rc, "dk_lora_grads_multi")
    return res


class LoraSums:
    """The column sums (dA, dB) lora_dz_multi left to do, for linear_backward_dx_lora(sums=...)
    to carry on its GEMM launch.  .grads is [(dA, dB, dz), ...] as lora_grads_multi returns it;
    dA and dB hold their values once that GEMM has run."""

    def __init__(self, x, arr, m, k, r, n, keep, res):
        self.grads = res
        self._keep = keep
        self.c = _lib.SideLoraSumsC(_lib.ptr(x), m, k, r, arr, n)
        self._arr = arr


def lora_dz_multi(x, terms, outs=None):
    """The first half of lora_grads_multi (same arguments): dz of every term now; the column sums
    are returned as a LoraSums for the q|k|v dX GEMM to carry (linear_backward_dx_lora(...,
    sums=...)), which makes dA and dB bit-identical to lora_grads_multi's."""
    arr, m, k, r, dev, keep, res = _lora_grads_args(x, terms, outs)
    rc = _lib.lib().dk_lora_dz_multi(_lib.ptr(x), m, k, r, arr, len(terms), _lib.stream_handle(dev))
    _lib.check(rc, "dk_lora_dz_multi")
    return LoraSums(x, arr, m, k, r, len(terms), keep, res)


def gateup_swiglu_forward(x, w_gu, act=None, gu=None, save_gu=True, w16=None, side=None):
    """gate|up as one NF4 GEMM with the gated-SiLU epilogue.  w_gu is [2I, in] (gate rows then up
    rows).  Returns (act [M, I], gu [M, 2I] or None).  w16, side as in linear_forward_lora."""
    if side is not None and w16 is None:
        raise ValueError("a carried dequant (side) needs the fp16-weight form (w16)")
    _check16(x, "x")
    m = x.shape[0]
    inter = w_gu.rows // 2
    if x.shape[1] != w_gu.cols or w_gu.rows % 2:
        raise ValueError("gate|up weight does not match x")
    dev = x.device
    if act is None:
        act = torch.empty(m, inter, dtype=torch.float16, device=dev)
    _check16(act, "act", (m, inter))
    if not act.is_contiguous():
        raise ValueError("act must be contiguous")
    if save_gu and gu is None:
        gu = torch.empty(m, 2 * inter, dtype=torch.float16, device=dev)
    if gu is not None:
        _check16(gu, "gu", (m, 2 * inter))
        if not gu.is_contiguous():
            raise ValueError("gu must be contiguous")
    if w16 is not None:
        _check_w16(w16, w_gu)
        rc = _lib.lib().dk_h16_gateup_swiglu_fwd(_lib.ptr(x), x.stride(0), m, _lib.ptr(w16),
                                                 w_gu.rows, w_gu.cols, _lib.ptr(act), _lib.ptr(gu),
                                                 None, 0, _side(side), _lib.stream_handle(dev))
        _lib.check(rc, "dk_h16_gateup_swiglu_fwd")
        return act, gu
    ws, nbytes = _workspace(w_gu, m, _lib.DK_OP_GATEUP_SWIGLU_FWD, dev)
    rc = _lib.lib().dk_w4_gateup_swiglu_fwd(_lib.ptr(x), x.stride(0), m, w_gu.c_ref(), _lib.ptr(act),
                                            _lib.ptr(gu), _lib.ptr(ws), nbytes,
                                            _lib.stream_handle(dev))
    _lib.check(rc, "dk_w4_gateup_swiglu_fwd")
    return act, gu


def down_swiglu_backward(dh, w_down, gu, w16=None, side=None):
    """dact = fp16(dh W_down), then gu <- [dgate | dup] in place.  Returns gu.  w16, side as in
    linear_forward_lora."""
    if side is not None and w16 is None:
        raise ValueError("a carried dequant (side) needs the fp16-weight form (w16)")
    _check16(dh, "dh")
    _check16(gu, "gu", (dh.shape[0], 2 * w_down.cols))
    if dh.shape[1] != w_down.rows or not gu.is_contiguous():
        raise ValueError("down backward: shapes do not match")
    if w16 is not None:
        _check_w16(w16, w_down)
        rc = _lib.lib().dk_h16_down_swiglu_bwd(_lib.ptr(dh), dh.stride(0), dh.shape[0], _lib.ptr(w16),
                                               w_down.rows, w_down.cols, _lib.ptr(gu), None, 0,
                                               _side(side), _lib.stream_handle(dh.device))
        _lib.check(rc, "dk_h16_down_swiglu_bwd")
        return gu
    ws, nbytes = _workspace(w_down, dh.shape[0], _lib.DK_OP_DOWN_SWIGLU_BWD, dh.device)
    rc = _lib.lib().dk_w4_down_swiglu_bwd(_lib.ptr(dh), dh.stride(0), dh.shape[0], w_down.c_ref(),
                                          _lib.ptr(gu), _lib.ptr(ws), nbytes,
                                          _lib.stream_handle(dh.device))
    _lib.check(rc, "dk_w4_down_swiglu_bwd")
    return gu


class QLoRALinearFunction(torch.autograd.Function):
    """y = x W^T (+ bias) + s * (drop(x) A^T) B^T with a frozen NF4 W; gradients for x, A, B.
    The dropout keep-mask is an input (uint8 [M, in]), as in the reference's norm kernel."""

    @staticmethod
    def forward(ctx, x, lora_A, lora_B, w, bias, mask, keep_scale, lora_scale):
        a16 = lora_A.detach().half().contiguous()
        b16 = lora_B.detach().half().contiguous()
        z = lora_down(x, a16, mask, keep_scale)
        y = linear_forward(x, w, bias, z, b16, lora_scale)
        ctx.save_for_backward(x, z, a16, b16, mask if mask is not None else torch.empty(0))
        ctx.w, ctx.ks, ctx.s, ctx.has_mask = w, keep_scale, lora_scale, mask is not None
        ctx.dtypes = (lora_A.dtype, lora_B.dtype)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, z, a16, b16, mask = ctx.saved_tensors
        mask = mask if ctx.has_mask else None
        dy = dy.contiguous().half()
        da, db, dz = lora_grads(dy, z, x, b16, ctx.s, mask, ctx.ks)
        dx = linear_backward_dx(dy, ctx.w, dz, a16, mask, ctx.ks, out_dtype=torch.float32)
        return (dx.to(x.dtype), da.to(ctx.dtypes[0]), db.to(ctx.dtypes[1]),
                None, None, None, None, None)


class QLoRALinear(torch.nn.Module):
    """A frozen NF4 linear with a trainable rank-r LoRA (A kaiming-uniform, B given or zero)."""

    def __init__(self, w, rank=16, alpha=32, dropout=0.05, bias=None):
        super().__init__()
        self.w = w
        self.bias = bias
        self.lora_A = torch.nn.Parameter(torch.empty(rank, w.cols, dtype=torch.float32, device=w.device))
        self.lora_B = torch.nn.Parameter(torch.zeros(w.rows, rank, dtype=torch.float32, device=w.device))
        torch.nn.init.kaiming_uniform_(self.lora_A, a=5 ** 0.5)
        self.scale = alpha / rank
        self.p = dropout
        self.keep_scale = 1.0 / float(torch.tensor(1.0 - dropout, dtype=torch.float32))

    def forward(self, x, mask=None):
        if mask is None and self.training and self.p > 0:
            mask = (torch.rand(x.shape, device=x.device) >= self.p).to(torch.uint8)
        ks = self.keep_scale if mask is not None else 1.0
        return QLoRALinearFunction.apply(x, self.lora_A, self.lora_B, self.w, self.bias, mask, ks,
                                         self.scale)


def default_tables(device):
    """(code2, nf4) fp32 tables on `device`."""
    return code2_on(device), nf4_table(device)
