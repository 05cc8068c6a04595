"""NF4 double-quantised weights: the repacked layer format and the dequant operators.

Drop-in for the reference's solution/k_nf4.py (same names, arguments, layout and errors), with
the dequant running in the gfx950 kernel ``dk_nf4_dequant`` of libdk.so instead of a Triton
kernel.  For element e of a weight (even e in the high nibble of byte e // 2):

    absmax[q] = fp32(fp32(code2[qabs[q]] * scale2[q // 256]) + offset2[q // 256]),  q = e // 64
    out[e]    = fp16(NF4[nibble] * absmax[q])

bit-identical to the reference (solution/k_nf4.py:16-21, 40-57).

A repacked layer (solution/k_nf4.py:64-95) is one flat uint8 buffer
``[packed | qabs | scale2 fp32 | offset2 fp32]``, each section on a 64-byte boundary, holding
the seven weights of a decoder layer in the order q, k, v, o, gate, up, down.  The fused GEMMs
of ``w4linear`` read the same sections directly (``PackedLayer.weight``).  Host-memory
streaming (the reference's SlotView / WeightPipe) is not part of this build.
"""

import torch

from . import _lib
from .quant import NF4_CODE  # noqa: F401  (re-exported: the reference module exposes it)

QBLOCKS_PER_PROGRAM = 128   # first-level blocks per dequant workgroup (1024 chunks of 8 weights)
LAYER_WEIGHTS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
RANGE_ALIGN = 1024          # reference solution/k_nf4.py:190


class PackedLayer:
    """The repacked 4-bit weights of one decoder layer (reference solution/k_nf4.py:64-78)."""

    def __init__(self, flat, offsets, n_qblocks, segments):
        self.flat, self.offsets = flat, offsets
        self.n_qblocks = n_qblocks
        self.segments = segments          # name -> (start element, rows, cols)
        self.numel = n_qblocks * 64
        self.packed, self.qabs, self.scale2, self.offset2 = section_views(flat, offsets, n_qblocks)

    def weight(self, name, code2, nf4):
        """The NF4 weight `name` of this layer as the fused GEMMs' operand (views, no copy)."""
        from .w4linear import W4
        start, rows, cols = self.segments[name]
        return W4.from_sections(self.packed, self.qabs, self.scale2, self.offset2, start,
                                rows, cols, code2, nf4)

    def weights(self, names, code2, nf4):
        """Consecutive weights of the layer as one stacked operand (e.g. gate|up or q|k|v)."""
        from .w4linear import W4
        start, rows, cols = self.segments[names[0]]
        at = start + rows * cols
        for name in names[1:]:
            s, r, c = self.segments[name]
            if s != at or c != cols:
                raise ValueError(f"{names} are not contiguous in the layer")
            rows += r
            at += r * c
        return W4.from_sections(self.packed, self.qabs, self.scale2, self.offset2, start,
                                rows, cols, code2, nf4)


def section_layout(n_qblocks):
    """Byte offsets of the four sections and the total size of a flat layer buffer."""
    sizes = (n_qblocks * 32, n_qblocks, (n_qblocks // 256) * 4, (n_qblocks // 256) * 4)
    offs, at = [], 0
    for size in sizes:
        offs.append(at)
        at += -(-size // 64) * 64
    return tuple(offs), at


def section_views(flat, offsets, n_qblocks):
    o_pk, o_qa, o_s2, o_o2 = offsets
    n2 = n_qblocks // 256
    return (flat[o_pk:o_pk + n_qblocks * 32], flat[o_qa:o_qa + n_qblocks],
            flat[o_s2:o_s2 + 4 * n2].view(torch.float32),
            flat[o_o2:o_o2 + 4 * n2].view(torch.float32))


def _quant_parts(linear):
    """(packed uint8 data, QuantState) of a 4-bit linear, checked for the nested NF4 format
    (reference solution/k_nf4.py:98-114)."""
    weight = linear.weight
    state = getattr(weight, "quant_state", None)
    if state is None:
        state = getattr(linear, "quant_state", None)
    if state is None:
        raise ValueError("4-bit weight without quant_state")
    if getattr(state, "quant_type", None) != "nf4" or int(state.blocksize) != 64:
        raise ValueError(f"unsupported 4-bit format {state.quant_type}/{state.blocksize}")
    if not getattr(state, "nested", False) or state.state2 is None or int(state.state2.blocksize) != 256:
        raise ValueError("expected double quantisation (nested absmax, blocksize 256)")
    if weight.data.dtype != torch.uint8:
        raise ValueError(f"packed storage {weight.data.dtype}, expected uint8")
    if state.dtype != torch.float16:
        raise ValueError(f"quant_state dtype {state.dtype}, expected float16")
    return weight, state


def layer_numel(linears):
    """Number of 4-bit weights of a layer (sum over its seven matrices)."""
    total = 0
    for name in LAYER_WEIGHTS:
        _, state = _quant_parts(linears[name])
        total += int(state.shape[0]) * int(state.shape[1])
    return total


def repack_layer(linears, device, host=False, out=None):
    """Repack the seven 4-bit linears of a layer (dict name -> module) into one PackedLayer and
    re-point their tensors at views of it, so nothing is stored twice (reference
    solution/k_nf4.py:126-173).  host=True gives a pinned host buffer.  Returns
    (PackedLayer, code2 fp32)."""
    parts = [(name, *_quant_parts(linears[name])) for name in LAYER_WEIGHTS]
    total = 0
    segments = {}
    code2 = None
    for name, weight, state in parts:
        rows, cols = int(state.shape[0]), int(state.shape[1])
        n = rows * cols
        if n % (64 * 256) != 0:
            raise ValueError(f"{name}: {n} weights do not fill whole absmax blocks")
        if weight.data.numel() * 2 != n or state.absmax.numel() * 64 != n:
            raise ValueError(f"{name}: unexpected packed sizes")
        if state.state2.absmax.numel() * 256 * 64 != n:
            raise ValueError(f"{name}: unexpected second-level absmax size")
        if code2 is None:
            code2 = state.state2.code.to(device)
        elif not torch.equal(code2, state.state2.code.to(device)):
            raise ValueError("second-level code tables differ between weights")
        segments[name] = (total, rows, cols)
        total += n
    n_qblocks = total // 64
    offsets, nbytes = section_layout(n_qblocks)
    if out is not None:
        if out.numel() != nbytes or out.dtype != torch.uint8:
            raise ValueError("preallocated layer buffer has the wrong size")
        flat = out
    elif host:
        flat = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    else:
        flat = torch.empty(nbytes, dtype=torch.uint8, device=device)
    packed, qabs, scale2, offset2 = section_views(flat, offsets, n_qblocks)
    for name, weight, state in parts:
        start, rows, cols = segments[name]
        n = rows * cols
        b0, q0, s0 = start // 2, start // 64, start // (64 * 256)
        b1, q1, s1 = b0 + n // 2, q0 + n // 64, s0 + n // (64 * 256)
        packed[b0:b1].copy_(weight.data.reshape(-1))
        qabs[q0:q1].copy_(state.absmax.reshape(-1))
        scale2[s0:s1].copy_(state.state2.absmax.reshape(-1).float())
        offset2[s0:s1].copy_(state.offset.float().reshape(1).expand(s1 - s0))
        weight.data = packed[b0:b1].view(weight.data.shape)
        state.absmax = qabs[q0:q1].view(state.absmax.shape)
        state.state2.absmax = scale2[s0:s1].view(state.state2.absmax.shape)
        state.offset = state.offset.to("cpu" if host else device)
    return PackedLayer(flat, offsets, n_qblocks, segments), code2.float().contiguous()


def dequant_tensors(packed, qabs, scale2, offset2, n_qblocks, code2, nf4, out):
    """Dequantise n_qblocks first-level blocks into the fp16 tensor `out` on the current stream
    (reference solution/k_nf4.py:176-181)."""
    n_qblocks = int(n_qblocks)
    for t, dt in ((packed, torch.uint8), (qabs, torch.uint8), (scale2, torch.float32),
                  (offset2, torch.float32), (code2, torch.float32), (nf4, torch.float32),
                  (out, torch.float16)):
        if t.dtype != dt or not t.is_cuda:
            raise ValueError(f"dequant operand has dtype {t.dtype} on {t.device}, expected CUDA {dt}")
    if (packed.numel() < n_qblocks * 32 or qabs.numel() < n_qblocks or out.numel() < n_qblocks * 64
            or scale2.numel() < -(-n_qblocks // 256) or offset2.numel() < -(-n_qblocks // 256)):
        raise ValueError("dequant operands are smaller than n_qblocks")
    rc = _lib.lib().dk_nf4_dequant(_lib.ptr(packed), _lib.ptr(qabs), _lib.ptr(scale2),
                                   _lib.ptr(offset2), _lib.ptr(code2), _lib.ptr(nf4),
                                   _lib.ptr(out), n_qblocks, _lib.stream_handle(out.device))
    _lib.check(rc, "dk_nf4_dequant")
    return out


def dequant_layer(layer, code2, nf4, out):
    """Dequantise every weight of `layer` (GPU-resident) into the flat fp16 buffer `out`."""
    return dequant_tensors(layer.packed, layer.qabs, layer.scale2, layer.offset2, layer.n_qblocks,
                           code2, nf4, out)


def side_dequant(layer, code2, nf4, out, sb0, sb1, wgs):
    """The dk_side_dequant a fp16-weight GEMM launch carries (w4linear's ``side=`` argument):
    second-level blocks [sb0, sb1) of `layer` (GPU-resident) into the whole-layer fp16 buffer
    `out` (weight e at out[e]), on `wgs` extra workgroups of the launch (-1: as many as the CUs
    its last round of tiles leaves idle, at least 16).  This is the reference's
    dequant ahead of use (dequant_range on dq_stream, solution/fast_qwen.py:729-731) moved into
    the launch of the GEMM it overlaps.  Returns the ctypes struct; `layer`, `out` and the tables
    must outlive the launch."""
    sb0, sb1, wgs = int(sb0), int(sb1), int(wgs)
    n_sb = layer.n_qblocks // 256
    if not (0 <= sb0 <= sb1 <= n_sb) or not (wgs == -1 or 0 <= wgs <= 1024):
        raise ValueError(f"side dequant of blocks [{sb0}, {sb1}) of {n_sb} on {wgs} workgroups")
    for t, dt in ((layer.packed, torch.uint8), (layer.qabs, torch.uint8),
                  (layer.scale2, torch.float32), (layer.offset2, torch.float32),
                  (code2, torch.float32), (nf4, torch.float32), (out, torch.float16)):
        if t.dtype != dt or not t.is_cuda:
            raise ValueError(f"dequant operand has dtype {t.dtype} on {t.device}, expected CUDA {dt}")
    if out.numel() < layer.n_qblocks * 64 or not out.is_contiguous():
        raise ValueError("side dequant output is not a contiguous whole-layer buffer")
    return _lib.SideDequantC(_lib.ptr(layer.packed), _lib.ptr(layer.qabs), _lib.ptr(layer.scale2),
                             _lib.ptr(layer.offset2), _lib.ptr(code2), _lib.ptr(nf4),
                             _lib.ptr(out), sb0, sb1, wgs)


def dequant_range(layer, q0, q1, code2, nf4, out, dst=None):
    """Dequantise first-level blocks [q0, q1) of `layer` into `out` at their own position, or at
    element offset `dst`.  q0 and q1 must be multiples of RANGE_ALIGN (q1 may be the layer end)
    and dst a multiple of RANGE_ALIGN * 64, else ValueError (reference
    solution/k_nf4.py:193-205)."""
    if q0 % RANGE_ALIGN or (q1 % RANGE_ALIGN and q1 != layer.n_qblocks):
        raise ValueError("dequant range not aligned")
    s0, s1 = q0 // 256, -(-q1 // 256)
    start = q0 * 64 if dst is None else int(dst)
    if start % (RANGE_ALIGN * 64):
        raise ValueError("dequant destination not aligned")
    return dequant_tensors(layer.packed[q0 * 32:q1 * 32], layer.qabs[q0:q1], layer.scale2[s0:s1],
                           layer.offset2[s0:s1], q1 - q0, code2, nf4,
                           out[start:start + (q1 - q0) * 64])


def warmup_specs():
    """Nothing to warm up: the kernels are compiled ahead of time into libdk.so."""
    return []
