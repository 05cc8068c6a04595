"""CPU check of the dequant-ahead schedule (decentrik_prime_amd/schedule.py, stack.py), the
counterpart of the reference's schedule check (dev/test_ws_schedule.py:102-235): the stack's real
step() runs against a model of HIP streams and events in which every launch is a node and a
stream's launches depend on its previous launch and on the events it waited for.  For several
steps of forward + backward, in every schedule (whole layer or per weight kind, in order or on a
side stream) it checks that

  * every GEMM reads slot contents dequantised from the layer and weight it multiplies, by the
    last dequant into that slot ordered before it, with no dequant into that slot unordered
    against it (no stale or racing read);
  * every dequant into a slot is ordered after every read of the slot's previous contents (no
    overwrite while in use);
  * the dequant count per step: 2 per layer, less the two layers still resident at the
    forward/backward turn and between steps (54 of 56 for 28 layers).
"""

import types

import pytest
import torch

from decentrik_prime_amd import k_nf4, stack as stack_mod
from decentrik_prime_amd.schedule import DequantAhead
from decentrik_prime_amd.stack import NF4LinearStack


class _Node:
    def __init__(self, what, deps):
        self.what, self.deps = what, deps


class _Streams:
    """Streams and events as a dependency graph of launches."""

    def __init__(self):
        self.nodes = []
        self.main = _Stream(self, "main")
        self.cur = self.main

    def before(self, a, b):
        """a is ordered before b."""
        seen, todo = set(), [b]
        while todo:
            x = todo.pop()
            for d in x.deps:
                if d is a:
                    return True
                if id(d) not in seen:
                    seen.add(id(d))
                    todo.append(d)
        return False


class _Stream:
    def __init__(self, g, name):
        self.g, self.name, self.last, self.waits = g, name, None, []

    def launch(self, what):
        node = _Node(what, ([self.last] if self.last else []) + self.waits)
        self.waits = []
        self.last = node
        self.g.nodes.append(node)
        return node

    def wait_event(self, ev):
        if ev.node is not None:
            self.waits.append(ev.node)


class _Event:
    def __init__(self, g):
        self.g, self.node = g, None

    def record(self, stream=None):
        self.node = (stream or self.g.cur).launch(("record",))


class _StreamCtx:
    def __init__(self, g, s):
        self.g, self.s = g, s

    def __enter__(self):
        self.prev, self.g.cur = self.g.cur, self.s

    def __exit__(self, *exc):
        self.g.cur = self.prev


class _W4:
    def __init__(self, g, layer, kind, n):
        self.g, self.layer, self.kind = g, layer, kind
        self.rows, self.cols = n, 1

    def dequantize(self, out):
        self.g.cur.launch(("write", _slot(out), (self.layer, self.kind)))
        return out


class _Packed:
    def __init__(self, layer, segments, numel):
        self.layer, self.segments, self.numel = layer, segments, numel


def _slot(t):
    return t.untyped_storage().data_ptr()


# a layer of 72 weights: q|k|v 16 at 0, o 8 at 16, gate|up 32 at 24, down 16 at 56
_SIZES = {"qkv": (0, 16), "o": (16, 8), "gu": (24, 32), "d": (56, 16)}
_FIRST = {"q_proj": "qkv", "o_proj": "o", "gate_proj": "gu", "down_proj": "d"}


def _fake_stack(g, n_layers, ahead, where):
    st = object.__new__(NF4LinearStack)
    st.n_layers, st.m, st.device = n_layers, 8, torch.device("cpu")
    st.s, st.keep_scale, st.probe = 2.0, 1.0, None
    st.code2 = st.nf4 = None
    segments = {name: (_SIZES[k][0], _SIZES[k][1], 1) for name, k in _FIRST.items()}
    st.layers = [dict(packed=_Packed(i, segments, 72),
                      **{k: _W4(g, i, k, n) for k, (_, n) in _SIZES.items()})
                 for i in range(n_layers)]
    st.lora = [dict(Aq=0, Av=0, Bq=0, Bv=0, mq=0, mv=0, bias=0) for _ in range(n_layers)]
    st.z = [dict(q=0, v=0) for _ in range(n_layers)]
    st.x, st.act = 0, 0
    st.dy = {"qkv": torch.zeros(8, 2048), "o": 0, "d": 0}
    st.out = {"qkv": 0, "o": 0, "y": 0}
    st.gu = [0] * n_layers
    st.dx_qkv = st.dx_o = st.dx_mlp = 0
    st.grads = [None] * n_layers
    st._setup_schedule(ahead, where)
    return st


def _gemm(g):
    def run(*args, **kwargs):
        w = next(a for a in args if isinstance(a, _W4))
        w16 = kwargs.get("w16")
        assert w16 is not None, "every GEMM reads a dequantised slot in these schedules"
        g.cur.launch(("read", _slot(w16), (w.layer, w.kind), w16.storage_offset()))
    return run


@pytest.fixture
def model(monkeypatch):
    g = _Streams()
    cuda = types.SimpleNamespace(
        Stream=lambda device=None: _Stream(g, "side"), Event=lambda **kw: _Event(g),
        stream=lambda s: _StreamCtx(g, s), current_stream=lambda device=None: g.cur)
    monkeypatch.setattr(torch, "cuda", cuda)
    for name in ("linear_forward_lora", "linear_forward", "gateup_swiglu_forward",
                 "down_swiglu_backward", "linear_backward_dx", "linear_backward_dx_lora"):
        monkeypatch.setattr(stack_mod, name, _gemm(g))
    monkeypatch.setattr(stack_mod, "lora_down_multi", lambda *a, **k: [0, 0])
    monkeypatch.setattr(stack_mod, "lora_grads_multi", lambda *a, **k: [(0, 0, 0), (0, 0, 0)])

    def dequant_layer(layer, code2, nf4, out):
        g.cur.launch(("write", _slot(out), (layer.layer, "layer")))
    monkeypatch.setattr(k_nf4, "dequant_layer", dequant_layer)
    return g


def _check(g, n_layers, steps, whole_layer):
    reads = [n for n in g.nodes if n.what[0] == "read"]
    writes = [n for n in g.nodes if n.what[0] == "write"]
    assert len(reads) == steps * n_layers * 8
    for r in reads:
        _, slot, (layer, kind), offset = r.what
        mine = [w for w in writes if w.what[1] == slot]
        ordered = [w for w in mine if g.before(w, r)]
        assert all(g.before(w, r) or g.before(r, w) for w in mine), f"dequant races a read of {kind}"
        last = [w for w in ordered if not any(g.before(w, x) for x in ordered if x is not w)]
        assert len(last) == 1
        wl, wk = last[0].what[2]
        assert wl == layer and wk == ("layer" if whole_layer else kind), \
            f"layer {layer} {kind} read slot contents of layer {wl} {wk}"
        if whole_layer:
            assert offset == _SIZES[kind][0]
    # no overwrite while in use: a write is ordered after every read of the previous contents
    for w in writes:
        for r in reads:
            if r.what[1] == w.what[1] and not g.before(w, r) and \
                    (r.what[2][0], "layer" if whole_layer else r.what[2][1]) != w.what[2]:
                assert g.before(r, w), "a dequant overwrites a slot another GEMM still reads"


@pytest.mark.parametrize("ahead", ["layer", ("qkv", "o", "gu", "d")])
@pytest.mark.parametrize("where", ["main", "side"])
def test_dequant_ahead_schedule(model, ahead, where):
    n_layers, steps = 5, 3
    st = _fake_stack(model, n_layers, ahead, where)
    per_step = []
    for _ in range(steps):
        before = sum(1 for n in model.nodes if n.what[0] == "write")
        st.step()
        per_step.append(sum(1 for n in model.nodes if n.what[0] == "write") - before)
    _check(model, n_layers, steps, ahead == "layer")
    kinds = 1 if ahead == "layer" else 4
    # the first step dequantises layer 0 on first use; every later step reuses the resident
    # last layer at the turn and layer 0 from the previous backward
    assert per_step[0] == kinds * (2 * n_layers - 1)
    assert per_step[1:] == [kinds * (2 * n_layers - 2)] * (steps - 1)
    if where == "side":
        assert any(n.deps and any(d is not None for d in n.deps) for n in model.nodes)


def test_model_catches_a_missing_wait(model, monkeypatch):
    """A planted mistake: take() that does not wait for the dequant makes the side-stream
    schedule race, and the check says so."""
    monkeypatch.setattr(DequantAhead, "take",
                        lambda self, kind, key: self.buf[kind][:self.numel[kind]])
    st = _fake_stack(model, 3, "layer", "side")
    st.step()
    with pytest.raises(AssertionError):
        _check(model, 3, 1, True)
