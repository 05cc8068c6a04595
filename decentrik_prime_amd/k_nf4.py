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

import itertools

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


# The format a 4-bit linear must have to be repacked (bitsandbytes NF4 with double quantisation,
# solution/k_nf4.py:98-114): each rule is (test of (weight, quant_state), what it requires).
_FORMAT_RULES = (
    (lambda w, s: getattr(s, "quant_type", None) == "nf4" and int(s.blocksize) == 64,
     "NF4 codes in first-level blocks of 64"),
    (lambda w, s: bool(getattr(s, "nested", False)) and s.state2 is not None
     and int(s.state2.blocksize) == 256,
     "an absmax double-quantised in second-level blocks of 256"),
    (lambda w, s: w.data.dtype == torch.uint8, "nibbles stored as uint8"),
    (lambda w, s: s.dtype == torch.float16, "a float16 dequantised dtype"),
)
_ELEMS_PER_SB = 64 * 256     # weights under one (scale2, offset2) entry


def _quant_parts(linear):
    """(Params4bit, QuantState) of a 4-bit linear whose format the repacked layer can hold; a
    ValueError names the first requirement it breaks (the reference's checks,
    solution/k_nf4.py:98-114)."""
    weight = linear.weight
    state = getattr(weight, "quant_state", None)
    if state is None:          # older bitsandbytes keeps the state on the module
        state = getattr(linear, "quant_state", None)
    if state is None:
        raise ValueError("the 4-bit weight carries no quant_state")
    for holds, requirement in _FORMAT_RULES:
        if not holds(weight, state):
            raise ValueError(f"4-bit weight format not supported: it must have {requirement}")
    return weight, state


def layer_numel(linears):
    """Number of 4-bit weights of a layer: the element counts of its seven matrices."""
    return sum(rows * cols for _, _, _, rows, cols in map(_source, LAYER_WEIGHTS,
                                                          (linears[n] for n in LAYER_WEIGHTS)))


def _source(name, linear):
    """(name, weight, state, rows, cols) of one linear, its section sizes checked against its
    shape: whole second-level blocks, n/2 packed bytes, n/64 and n/16384 absmax entries."""
    weight, state = _quant_parts(linear)
    rows, cols = (int(d) for d in state.shape)
    n = rows * cols
    sizes = {"whole second-level blocks": n % _ELEMS_PER_SB == 0,
             "packed bytes": 2 * weight.data.numel() == n,
             "first-level absmax entries": 64 * state.absmax.numel() == n,
             "second-level absmax entries": _ELEMS_PER_SB * state.state2.absmax.numel() == n}
    wrong = [what for what, ok in sizes.items() if not ok]
    if wrong:
        raise ValueError(f"{name}: a [{rows}, {cols}] weight with the wrong {', '.join(wrong)}")
    return name, weight, state, rows, cols


def _layer_buffer(nbytes, device, host, out):
    if out is None:
        where = {"pin_memory": True} if host else {"device": device}
        return torch.empty(nbytes, dtype=torch.uint8, **where)
    if out.dtype != torch.uint8 or out.numel() != nbytes:
        raise ValueError(f"the preallocated layer buffer must be {nbytes} uint8 bytes")
    return out


def repack_layer(linears, device, host=False, out=None):
    """Repack the seven 4-bit linears of a layer (dict name -> module) into one PackedLayer and
    re-point their tensors at views of it, so nothing is stored twice (reference
    solution/k_nf4.py:126-173).  host=True gives a pinned host buffer; `out` a preallocated one.
    Returns (PackedLayer, code2 fp32)."""
    sources = [_source(name, linears[name]) for name in LAYER_WEIGHTS]
    tables = [src[2].state2.code.to(device) for src in sources]
    if not all(torch.equal(tables[0], t) for t in tables[1:]):
        raise ValueError("the weights of a layer must share one second-level code table")
    starts = list(itertools.accumulate((rows * cols for *_, rows, cols in sources), initial=0))
    segments = {src[0]: (at, src[3], src[4]) for src, at in zip(sources, starts)}
    n_qblocks = starts[-1] // 64
    offsets, nbytes = section_layout(n_qblocks)
    layer = PackedLayer(_layer_buffer(nbytes, device, host, out), offsets, n_qblocks, segments)
    home = "cpu" if host else device
    for (name, weight, state, rows, cols), at in zip(sources, starts):
        n = rows * cols
        # this weight's run of each section: bytes, first-level blocks, second-level blocks
        nib = layer.packed.narrow(0, at // 2, n // 2)
        first = layer.qabs.narrow(0, at // 64, n // 64)
        scale2 = layer.scale2.narrow(0, at // _ELEMS_PER_SB, n // _ELEMS_PER_SB)
        offset2 = layer.offset2.narrow(0, at // _ELEMS_PER_SB, n // _ELEMS_PER_SB)
        nib.copy_(weight.data.flatten())
        first.copy_(state.absmax.flatten())
        scale2.copy_(state.state2.absmax.flatten())
        # bitsandbytes keeps one offset per weight; the format has one per second-level block
        offset2.copy_(torch.broadcast_to(state.offset.float().reshape(()), offset2.shape))
        weight.data = nib.view(weight.data.shape)
        state.absmax = first.view(state.absmax.shape)
        state.state2.absmax = scale2.view(state.state2.absmax.shape)
        state.offset = state.offset.to(home)
    return layer, tables[0].float().contiguous()


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
