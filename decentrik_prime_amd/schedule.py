"""Dequant-ahead schedule: NF4 weights dequantised to fp16 on a side stream before the GEMM that
reads them.

Mirrors the reference's workspace schedule (solution/fast_qwen.py:694-756: ``_ws_load`` issues
``k_nf4.dequant_range`` into a workspace region on ``dq_stream`` with events ordering it after the
region's last reader and before its next one).  Here each weight kind has one fp16 slot; the
dequant kernel (HBM-bound) runs on the side stream while the compute-bound GEMMs of the preceding
operators run on the current stream.  A slot remembers which weight it holds, so a weight needed
again while still resident (the last layer at the forward/backward turn, the first layer at the
next step) is not dequantised twice.  Both streams keep the default priority.
"""

import torch


class DequantAhead:
    """One fp16 slot per weight kind, filled on ``self.stream`` and read on the current stream."""

    def __init__(self, device, sizes, stream="side"):
        """sizes: {kind: number of fp16 elements of the largest weight of that kind}.  stream:
        "side" for a stream of its own (default priority), "main" to dequantise in order on the
        current stream, or a torch stream to use."""
        self.device = torch.device(device)
        if stream == "side":
            stream = torch.cuda.Stream(self.device)
        elif stream == "main":
            stream = None
        self.stream = stream
        self.buf = {k: torch.empty(n, dtype=torch.float16, device=self.device)
                    for k, n in sizes.items()}
        self.holds = {k: None for k in sizes}     # key of the weight in the slot
        self.numel = {k: 0 for k in sizes}        # its element count
        self.ready = {k: None for k in sizes}     # event: the slot's dequant has finished
        self.free = {k: None for k in sizes}      # event: the slot's last reader was issued

    def issue(self, kind, key, w4):
        """Dequantise W4 weight ``w4`` (identified by ``key``) into slot ``kind`` on the side stream,
        after the slot's last reader; no-op when the slot already holds it."""
        if self.holds[kind] == key:
            return
        n = w4.rows * w4.cols
        if n > self.buf[kind].numel():
            raise ValueError(f"{kind}: a {w4.rows} x {w4.cols} weight does not fit the slot")
        out = self.buf[kind][:n]
        if self.stream is None:
            w4.dequantize(out=out.view(w4.rows, w4.cols))
            ev = None
        else:
            with torch.cuda.stream(self.stream):
                if self.free[kind] is not None:
                    self.stream.wait_event(self.free[kind])
                w4.dequantize(out=out.view(w4.rows, w4.cols))
                ev = torch.cuda.Event()
                ev.record(self.stream)
        self.ready[kind] = ev
        self.holds[kind] = key
        self.numel[kind] = n

    def take(self, kind, key):
        """The slot's fp16 weight, with the current stream ordered after its dequant."""
        if self.holds[kind] != key:
            raise RuntimeError(f"slot {kind} holds {self.holds[kind]}, not {key}")
        if self.ready[kind] is not None:
            torch.cuda.current_stream(self.device).wait_event(self.ready[kind])
        return self.buf[kind][:self.numel[kind]]

    def release(self, kind):
        """Mark the slot's last reader issued on the current stream (a later issue waits for it)."""
        if self.stream is None:
            return
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self.free[kind] = ev
