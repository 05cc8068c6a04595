"""NF4 double quantisation on the GPU, producing bitsandbytes-shaped weight objects.

The reference receives its 4-bit weights from bitsandbytes (``Params4bit`` with
``quant_type="nf4", compress_statistics=True, blocksize=64``) and reads them through
``weight.data`` (packed uint8) and ``weight.quant_state`` (solution/k_nf4.py:98-114).  This module
supplies objects with exactly those attributes, so ``k_nf4.repack_layer`` works on them as the
reference's does on bitsandbytes modules, and quantises on the GPU with ``dk_nf4_quantize``:

    absmax   = max |w| per 64 weights
    code     = number of fp32 NF4 midpoints strictly below w * fp32(1 / absmax)   (hi nibble first)
    offset   = mean(absmax), formed exactly (integer sum in units of 2^-24) and rounded to fp32
    qabs     = nearest entry of the signed dynamic map to (absmax - offset) / max|block of 256|
    absmax2  = max |absmax - offset| per 256 first-level blocks

The thresholds and the tie rules are this build's own; bitsandbytes is not installed here, so
whether its quantiser picks the same codes is not pinned.  The dequantised value of whatever codes
are stored is exact (the dequant closed form does not depend on how the codes were chosen).
"""

import numpy as np
import torch

from . import _lib

NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)

BLOCKSIZE = 64
BLOCKSIZE2 = 256


def dynamic_map_signed():
    """bitsandbytes' signed 8-bit dynamic map (create_dynamic_map(signed=True)), as fp32 [256]:
    for decades i = 0..6 the midpoints of 2**i + 1 evenly spaced points in [0.1, 1] scaled by
    10**(i - 6), both signs, plus 0 and 1, sorted."""
    vals = [0.0, 1.0]
    for i in range(7):
        pts = np.linspace(0.1, 1.0, 2 ** i + 1, dtype=np.float32)
        mids = ((pts[:-1] + pts[1:]) / np.float32(2.0)).astype(np.float32)
        scaled = (np.float32(10.0 ** (i - 6)) * mids).astype(np.float32)
        vals += scaled.tolist() + (-scaled).tolist()
    return torch.tensor(sorted(vals), dtype=torch.float32)


class QuantState:
    """The attributes of bitsandbytes' QuantState that the NF4 path reads."""

    def __init__(self, absmax, shape, code, blocksize, quant_type, dtype, offset=None, state2=None):
        self.absmax = absmax
        self.shape = torch.Size(shape)
        self.code = code
        self.blocksize = blocksize
        self.quant_type = quant_type
        self.dtype = dtype
        self.offset = offset
        self.state2 = state2
        self.nested = state2 is not None


class Params4bit:
    """A packed 4-bit weight: ``data`` is uint8 [numel / 2, 1], ``quant_state`` its QuantState."""

    def __init__(self, data, quant_state):
        self.data = data
        self.quant_state = quant_state
        self.requires_grad = False


class Linear4bit(torch.nn.Module):
    """A frozen NF4 linear layer with the attribute layout of bitsandbytes' Linear4bit."""

    def __init__(self, weight, bias=None):
        super().__init__()
        self.weight = weight
        self.bias = bias


_CODE2 = {}


def code2_on(device):
    device = torch.device(device)
    t = _CODE2.get(device)
    if t is None:
        t = _CODE2[device] = dynamic_map_signed().to(device)
    return t


def nf4_table(device):
    return torch.tensor(NF4_CODE, dtype=torch.float32, device=device)


def quantize_into(w16, code2, nf4, packed, qabs, scale2, offset2):
    """Quantise the fp16 CUDA tensor ``w16`` into caller-provided section views (the four sections
    of a repacked layer, or standalone tensors)."""
    n = w16.numel()
    if w16.dtype != torch.float16 or not w16.is_cuda or not w16.is_contiguous():
        raise ValueError("expected a contiguous fp16 CUDA tensor")
    if n % (BLOCKSIZE * BLOCKSIZE2):
        raise ValueError(f"{n} weights do not fill whole second-level blocks")
    for t, size in ((packed, n // 2), (qabs, n // 64), (scale2, n // 16384), (offset2, n // 16384)):
        if t.numel() != size:
            raise ValueError("section size mismatch")
    absmax_ws = torch.empty(n // 64, dtype=torch.float32, device=w16.device)
    sum_ws = torch.empty(1, dtype=torch.int64, device=w16.device)
    rc = _lib.lib().dk_nf4_quantize(
        _lib.ptr(w16), n, _lib.ptr(code2), _lib.ptr(nf4), _lib.ptr(packed), _lib.ptr(qabs),
        _lib.ptr(scale2), _lib.ptr(offset2), _lib.ptr(absmax_ws), _lib.ptr(sum_ws),
        _lib.stream_handle(w16.device))
    _lib.check(rc, "dk_nf4_quantize")
    return absmax_ws, sum_ws


def quantize_4bit(w16, code2=None):
    """NF4 + double quantisation of an fp16 CUDA weight [rows, cols] -> Params4bit."""
    dev = w16.device
    code2 = code2_on(dev) if code2 is None else code2
    nf4 = nf4_table(dev)
    n = w16.numel()
    packed = torch.empty(n // 2, dtype=torch.uint8, device=dev)
    qabs = torch.empty(n // 64, dtype=torch.uint8, device=dev)
    scale2 = torch.empty(n // 16384, dtype=torch.float32, device=dev)
    offset2 = torch.empty(n // 16384, dtype=torch.float32, device=dev)
    quantize_into(w16.contiguous(), code2, nf4, packed, qabs, scale2, offset2)
    state2 = QuantState(scale2, (n // 64,), code2, BLOCKSIZE2, "dynamic", torch.float32)
    qs = QuantState(qabs, tuple(w16.shape), nf4, BLOCKSIZE, "nf4", torch.float16,
                    offset=offset2[:1].clone(), state2=state2)
    return Params4bit(packed.view(-1, 1), qs)
