"""CPU check of the dequant-ahead schedule (decentrik_prime_amd/schedule.py, stack.py), the
counterpart of the reference's schedule check (dev/test_ws_schedule.py:102-235): the stack's real
step() runs against a model of HIP streams and events in which every launch is a node and a
stream's launches depend on its previous launch and on the events it waited for.  A launch reads
and writes fp16 slot memory in units of one second-level block (16384 weights).  For several
steps of forward + backward, in every schedule (per weight kind or whole layer, in order or on a
side stream, or carried by the GEMM launches into two alternating slots) it checks that

  * every GEMM reads, in each unit of its weight, what the last write ordered before it put
    there, and that write dequantised the layer the GEMM multiplies, with no write of that unit
    unordered against the read (no stale or racing read);
  * no write of a unit is unordered against a read of the unit (no overwrite while in use);
  * the dequant work per step: every layer twice, less the two layers still resident at the
    forward/backward turn and between steps (54 of 56 for 28 layers), in every schedule.
"""

import types

import pytest
import torch

from decentrik_prime_amd import k_nf4, stack as stack_mod
from decentrik_prime_amd.schedule import DequantAhead
from decentrik_prime_amd.stack import NF4LinearStack

UNIT = 16384   # weights per second-level block


class _Node:
    def __init__(self, acts, deps):
        self.acts, self.deps = acts, deps


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

    def acts(self, kind):
        return [(n, a) for n in self.nodes for a in n.acts if a[0] == kind]


class _Stream:
    def __init__(self, g, name):
        self.g, self.name, self.last, self.waits = g, name, None, []

    def launch(self, *acts):
        node = _Node(list(acts), ([self.last] if self.last else []) + self.waits)
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


def _units(t, lo=0, n=None):
    """(storage, frozenset of units) of elements [lo, lo + n) of the flat tensor t."""
    n = t.numel() if n is None else n
    first = t.storage_offset() + lo
    assert first % UNIT == 0 and n % UNIT == 0
    return t.untyped_storage().data_ptr(), frozenset(range(first // UNIT, (first + n) // UNIT))


class _W4:
    def __init__(self, g, layer, kind, n):
        self.g, self.layer, self.kind = g, layer, kind
        self.rows, self.cols = n, 1

    def dequantize(self, out):
        self.g.cur.launch(("write",) + _units(out) + ((self.layer, self.kind),))
        return out


class _Packed:
    def __init__(self, layer, segments, numel):
        self.layer, self.segments, self.numel = layer, segments, numel
        self.n_qblocks = numel // 64


# a layer of 8 units: q|k|v 2 at 0, o 1 at 2, gate|up 3 at 3, down 2 at 6
_SIZES = {"qkv": (0, 2 * UNIT), "o": (2 * UNIT, UNIT), "gu": (3 * UNIT, 3 * UNIT), "d": (6 * UNIT, 2 * UNIT)}
_FIRST = {"q_proj": "qkv", "o_proj": "o", "gate_proj": "gu", "down_proj": "d"}
_LAYER_UNITS = 8


def _fake_stack(g, n_layers, ahead, where):
    st = object.__new__(NF4LinearStack)
    st.n_layers, st.m, st.device = n_layers, 8, torch.device("cpu")
    st.s, st.keep_scale, st.probe = 2.0, 1.0, None
    st.code2 = st.nf4 = None
    segments = {name: (_SIZES[k][0], _SIZES[k][1], 1) for name, k in _FIRST.items()}
    st.layers = [dict(packed=_Packed(i, segments, _LAYER_UNITS * UNIT),
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


class _Side:
    """What k_nf4.side_dequant describes: blocks [sb0, sb1) of a layer into a whole-layer slot."""

    def __init__(self, layer, code2, nf4, out, sb0, sb1, wgs):
        assert wgs == -1 or wgs > 0
        self.act = ("write",) + _units(out, sb0 * UNIT, (sb1 - sb0) * UNIT) + ((layer.layer, "layer"),)


def _gemm(g):
    def run(*args, **kwargs):
        w = next(a for a in args if isinstance(a, _W4))
        w16 = kwargs.get("w16")
        assert w16 is not None, "every GEMM reads a dequantised slot in these schedules"
        side = kwargs.get("side")
        acts = [("read",) + _units(w16) + ((w.layer, w.kind), w16.storage_offset())]
        if side is not None:
            acts.append(side.act)
        g.cur.launch(*acts)
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
    def lora_down_multi(*args, dequant=None, **kwargs):
        # (the downs touch no slot memory) with a dequant (k_nf4.side_dequant), the launch writes
        # the dequant's blocks
        if dequant is not None:
            g.cur.launch(dequant.act).lora = True
        return [0, 0]
    monkeypatch.setattr(stack_mod, "lora_down_multi", lora_down_multi)
    monkeypatch.setattr(stack_mod, "lora_grads_multi", lambda *a, **k: [(0, 0, 0), (0, 0, 0)])
    monkeypatch.setattr(stack_mod, "lora_dz_multi",
                        lambda *a, **k: types.SimpleNamespace(grads=[(0, 0, 0), (0, 0, 0)]))

    def dequant_layer(layer, code2, nf4, out):
        g.cur.launch(("write",) + _units(out) + ((layer.layer, "layer"),))
    monkeypatch.setattr(k_nf4, "dequant_layer", dequant_layer)
    monkeypatch.setattr(k_nf4, "side_dequant", _Side)
    return g


def _check(g, n_layers, steps, whole_layer):
    reads = g.acts("read")
    writes = g.acts("write")
    assert len(reads) == steps * n_layers * 8
    for rn, (_, ptr, units, (layer, kind), offset) in reads:
        for u in units:
            mine = [(wn, w) for wn, w in writes if w[1] == ptr and u in w[2]]
            assert all(wn is not rn for wn, _ in mine), f"a launch writes the unit its GEMM reads"
            assert all(g.before(wn, rn) or g.before(rn, wn) for wn, _ in mine), \
                f"a dequant races the read of layer {layer} {kind}"
            ordered = [(wn, w) for wn, w in mine if g.before(wn, rn)]
            last = [(wn, w) for wn, w in ordered
                    if not any(g.before(wn, xn) for xn, _ in ordered if xn is not wn)]
            assert len(last) == 1
            wl, wk = last[0][1][3]
            assert wl == layer and wk == ("layer" if whole_layer else kind), \
                f"layer {layer} {kind} read unit {u} holding layer {wl} {wk}"
        if whole_layer:
            assert offset % (_LAYER_UNITS * UNIT) == _SIZES[kind][0]


def _units_written(g):
    return sum(len(w[2]) for _, w in g.acts("write"))


@pytest.mark.parametrize("ahead,where", [("layer", "main"), ("layer", "side"),
                                         (("qkv", "o", "gu", "d"), "main"),
                                         (("qkv", "o", "gu", "d"), "side"),
                                         ("carried", "main")])
def test_dequant_ahead_schedule(model, ahead, where):
    n_layers, steps = 5, 3
    st = _fake_stack(model, n_layers, ahead, where)
    per_step = []
    for _ in range(steps):
        before = _units_written(model)
        st.step()
        per_step.append((_units_written(model) - before) / _LAYER_UNITS)
    _check(model, n_layers, steps, ahead in ("layer", "carried"))
    # the first step dequantises layer 0 on first use; every later step reuses the resident
    # last layer at the turn and layer 0 from the previous backward
    assert per_step[0] == 2 * n_layers - 1
    assert per_step[1:] == [2 * n_layers - 2] * (steps - 1)
    if where == "side":
        assert any(len(n.deps) > 1 for n in model.nodes)


def test_forward_dequant_rides_on_the_lora_downs(model):
    """ahead="layer" on one stream: in the forward, every layer's dequant but the resident first
    one is the launch of that layer's LoRA downs (deferred from the previous layer's last GEMM);
    the backward's stay launches of their own."""
    n_layers = 4
    st = _fake_stack(model, n_layers, "layer", "main")
    st.step()
    first = len(model.nodes)
    st.step()
    later = model.nodes[first:]
    writes = [n for n in later if any(a[0] == "write" for a in n.acts)]
    riding = [n for n in writes if getattr(n, "lora", False)]
    assert len(riding) == n_layers - 1
    assert len(writes) == 2 * n_layers - 2
    assert sorted(n.acts[0][3][0] for n in riding) == list(range(1, n_layers))


def test_carried_dequant_rides_on_the_gemm_launches(model):
    """ahead="carried": every launch in the carry table writes the other slot's blocks of the next
    layer in step order; after the first step, the only dequant launches of their own are those of
    the layers no launch carries (the forward's, with an empty forward table)."""
    st = _fake_stack(model, 4, "carried", "main")
    st.step()
    first = len(model.nodes)
    st.step()
    later = model.nodes[first:]
    alone = [n for n in later if not any(a[0] == "read" for a in n.acts)]
    assert len(alone) == (0 if NF4LinearStack.CARRY["fwd"] else 3)
    carriers = [n for n in later if len(n.acts) == 2]
    n_fwd, n_bwd = len(NF4LinearStack.CARRY["fwd"]), len(NF4LinearStack.CARRY["bwd"])
    assert len(carriers) == 3 * n_fwd + 3 * n_bwd    # layers 0-2 forward, 3-1 backward
    for n in carriers:
        (_, rptr, _, (layer, _), _), (_, wptr, _, (wl, _)) = n.acts
        assert rptr != wptr and abs(wl - layer) == 1


def test_model_catches_a_missing_wait(model, monkeypatch):
    """A planted mistake: take() that does not wait for the dequant makes the side-stream
    schedule race, and the check says so."""
    monkeypatch.setattr(DequantAhead, "take",
                        lambda self, kind, key: self.buf[kind][:self.numel[kind]])
    st = _fake_stack(model, 3, "layer", "side")
    st.step()
    with pytest.raises(AssertionError):
        _check(model, 3, 1, True)


def test_model_catches_a_carry_into_the_slot_in_use(model, monkeypatch):
    """A planted mistake: carrying the next layer into the slot being read (one slot instead of
    two alternating ones) is caught."""
    st = _fake_stack(model, 3, "carried", "main")
    st.slots[1] = st.slots[0]
    st.step()
    with pytest.raises(AssertionError):
        _check(model, 3, 1, True)
