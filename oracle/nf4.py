"""CPU restatement of the NF4 double-quantised weight format.  TEST INFRASTRUCTURE ONLY.

Format (reference solution/k_nf4.py:16-21, bitsandbytes 0.50.2 nested NF4, blocksize 64/256):
element e of a weight lives in byte e // 2, the even element in the high nibble, and
dequantises to

    absmax[q] = fp32( fp32(code2[qabs[q]] * scale2[q // 256]) + offset2[q // 256] )   q = e // 64
    out[e]    = fp16_rne( fp32(NF4[nibble(e)] * absmax[q]) )

with the product and the sum rounded separately (no fused multiply-add), exactly as the reference
kernel computes it (solution/k_nf4.py:40-57) and as its NumPy check restates it
(dev/test_emu.py:48-55).

The quantiser below is this build's own bitsandbytes-style quantiser (blockwise absmax NF4,
then a blockwise 8-bit quantisation of absmax - mean(absmax) against the signed dynamic map).
bitsandbytes is not installed here, so the quantiser's parity with bitsandbytes is UNPINNED; it
only has to agree bit-exactly with the build's GPU quantiser.  Dequant parity does not depend
on it: the dequant is pinned by the closed form on identical packed inputs.
"""

import numpy as np

# NF4 code book (reference solution/k_nf4.py:28-34, bitsandbytes nf4_dequantization_lut).  A
# format constant: it must be identical, value for value, to the reference's table.
NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)

BLOCK = 64          # weights per first-level (NF4) block
BLOCK2 = 256        # first-level blocks per second-level block
RANGE_ALIGN = 1024  # reference solution/k_nf4.py:190
F32, F16 = np.float32, np.float16


def nf4_table():
    return np.array(NF4_CODE, dtype=F32)


def dynamic_map_signed():
    """The 256-entry signed dynamic code of bitsandbytes' blockwise 8-bit quantiser
    (functional.create_dynamic_map(signed=True, max_exponent_bits=7, total_bits=8)), restated:
    for each decade i = 0..6, the midpoints of 2**i + 1 evenly spaced points in [0.1, 1], scaled
    by 10**(i-6), with both signs; plus 0 and 1; sorted ascending."""
    vals = [0.0, 1.0]
    for i in range(7):
        pts = np.linspace(0.1, 1.0, 2 ** i + 1, dtype=np.float32)
        mids = (pts[:-1] + pts[1:]) / np.float32(2.0)
        scaled = (F32(10.0 ** (i - 6)) * mids).astype(F32)
        for m in scaled.tolist():
            vals.append(m)
            vals.append(-m)
    assert len(vals) == 256
    return np.array(sorted(vals), dtype=F32)


def nf4_midpoints():
    """Decision thresholds between consecutive NF4 codes, fp32((a + b) * 0.5)."""
    t = nf4_table()
    return ((t[:-1] + t[1:]) * F32(0.5)).astype(F32)


def _recip(a):
    """fp32 reciprocal with the convention that an all-zero block normalises to zero."""
    a = np.asarray(a, dtype=F32)
    out = np.zeros_like(a)
    nz = a != 0
    out[nz] = F32(1.0) / a[nz]
    return out


def quantize_nf4(w16):
    """First level: fp16 weights (flat, numel % 64 == 0) -> (packed uint8 [n/2], absmax fp32 [n/64]).
    code = number of NF4 midpoints strictly below w * fp32(1/absmax); byte = hi<<4 | lo."""
    w = np.asarray(w16, dtype=F16).reshape(-1)
    if w.size % BLOCK:
        raise ValueError("numel must be a multiple of 64")
    blocks = w.astype(F32).reshape(-1, BLOCK)
    absmax = np.abs(blocks).max(axis=1).astype(F32)
    x = (blocks * _recip(absmax)[:, None]).astype(F32)
    mids = nf4_midpoints()
    code = (x[..., None] > mids).sum(axis=-1).astype(np.uint8).reshape(-1)
    packed = ((code[0::2] << 4) | code[1::2]).astype(np.uint8)
    return packed, absmax


def exact_mean(absmax):
    """mean(absmax) rounded once to fp32.  Every absmax is the magnitude of an fp16 value, hence an
    integer multiple of 2**-24, so the sum is formed exactly in int64 units of 2**-24 (order
    independent) and divided in fp64."""
    a = np.asarray(absmax, dtype=F32).astype(np.float64)
    units = np.rint(a * 2.0 ** 24).astype(np.int64)
    if not np.array_equal(units.astype(np.float64) * 2.0 ** -24, a):
        raise ValueError("absmax values are not fp16 magnitudes")
    s = int(units.sum())
    return F32((np.float64(s) / np.float64(a.size)) * 2.0 ** -24)


def nearest_code(y, code):
    """Index of the nearest entry of the sorted table `code` (ties to the lower index)."""
    y = np.asarray(y, dtype=F32)
    lo = np.clip(np.searchsorted(code, y, side="right") - 1, 0, code.size - 1)
    hi = np.minimum(lo + 1, code.size - 1)
    d_hi = (code[hi] - y).astype(F32)
    d_lo = (y - code[lo]).astype(F32)
    return np.where(d_hi < d_lo, hi, lo).astype(np.uint8)


def double_quant(absmax, code2):
    """Second level: absmax fp32 [nq] (nq % 256 == 0) -> (qabs uint8 [nq], scale2 fp32 [nq/256],
    offset fp32 scalar)."""
    absmax = np.asarray(absmax, dtype=F32)
    if absmax.size % BLOCK2:
        raise ValueError("first-level block count must be a multiple of 256")
    offset = exact_mean(absmax)
    v = (absmax - offset).astype(F32).reshape(-1, BLOCK2)
    a2 = np.abs(v).max(axis=1).astype(F32)
    y = (v * _recip(a2)[:, None]).astype(F32)
    qabs = nearest_code(y.reshape(-1), np.asarray(code2, dtype=F32))
    return qabs, a2, offset


def quantize(w16, code2=None):
    """Whole bitsandbytes-style NF4 + double quant of one weight.  Returns a dict with the four
    sections the kernels read (offset2 broadcast per second-level block, as repack_layer does,
    reference solution/k_nf4.py:168)."""
    if code2 is None:
        code2 = dynamic_map_signed()
    packed, absmax = quantize_nf4(w16)
    qabs, scale2, offset = double_quant(absmax, code2)
    offset2 = np.full(scale2.shape, offset, dtype=F32)
    return dict(packed=packed, qabs=qabs, scale2=scale2, offset2=offset2, offset=offset,
                code2=np.asarray(code2, dtype=F32), absmax=absmax)


def absmax_of(qabs, scale2, offset2, code2):
    """fp32(fp32(code2[q] * scale2) + offset2), no fused multiply-add (solution/k_nf4.py:47-49)."""
    qabs = np.asarray(qabs, dtype=np.uint8)
    sb = np.arange(qabs.size) // BLOCK2
    first = (np.asarray(code2, F32)[qabs] * np.asarray(scale2, F32)[sb]).astype(F32)
    return (first + np.asarray(offset2, F32)[sb]).astype(F32)


def dequant(packed, qabs, scale2, offset2, code2, nf4=None):
    """The dequant closed form (solution/k_nf4.py:40-57): flat fp16 [2 * len(packed)]."""
    nf4 = nf4_table() if nf4 is None else np.asarray(nf4, dtype=F32)
    packed = np.asarray(packed, dtype=np.uint8)
    absmax = absmax_of(qabs, scale2, offset2, code2)
    blk = np.arange(packed.size) // (BLOCK // 2)
    out = np.empty(packed.size * 2, dtype=F16)
    out[0::2] = (nf4[packed >> 4] * absmax[blk]).astype(F32).astype(F16)
    out[1::2] = (nf4[packed & 15] * absmax[blk]).astype(F32).astype(F16)
    return out


def section_layout(n_qblocks):
    """Byte offsets of the four sections of a flat layer buffer and its size: packed | qabs |
    scale2 | offset2, each on a 64-byte boundary (reference solution/k_nf4.py:81-88)."""
    sizes = (n_qblocks * 32, n_qblocks, (n_qblocks // BLOCK2) * 4, (n_qblocks // BLOCK2) * 4)
    offs, at = [], 0
    for size in sizes:
        offs.append(at)
        at += -(-size // 64) * 64
    return tuple(offs), at


def dequant_range(packed, qabs, scale2, offset2, code2, q0, q1):
    """Dequant of quantisation blocks [q0, q1) (reference solution/k_nf4.py:193-205 rules)."""
    n_q = qabs.size
    if q0 % RANGE_ALIGN or (q1 % RANGE_ALIGN and q1 != n_q):
        raise ValueError("dequant range not aligned")
    s0, s1 = q0 // BLOCK2, -(-q1 // BLOCK2)
    return dequant(packed[q0 * 32:q1 * 32], qabs[q0:q1], scale2[s0:s1], offset2[s0:s1], code2)
