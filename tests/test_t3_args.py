"""The Python view's T3 wrappers check the tensors they hand to the C ABI as
raw addresses (cache shape against the model's layers and heads, dtypes,
contiguity, row counts) and raise ValueError before any call reaches the
library.  CPU only: the checks run on CPU tensors and a handle that was
never opened, so a call that got past them would fail on the missing
library handle instead of raising ValueError."""
import pytest

import pkg

torch = pytest.importorskip("torch")

NL, NH, NE, NCTX = 3, 4, 256, 32


def model(mod):
    m = mod.T3Model()
    m.n_layer, m.n_head, m.n_embd, m.n_pos = NL, NH, NE, NCTX
    return m


def unopened(mod):
    return object.__new__(mod.Sampler)  # no library handle


def good(rows=2, slots=None):
    slots = rows if slots is None else slots
    z = lambda *s, dt=torch.float32: torch.zeros(s, dtype=dt)
    return dict(k=z(slots, NL, NH, NCTX, 64), v=z(slots, NL, NH, NCTX, 64), h=z(rows, NE),
                pos=z(rows, dt=torch.int32), tok=z(rows, dt=torch.int32))


@pytest.mark.parametrize("bad", ["layers", "heads", "head_dim", "v_shape", "dtype", "noncontig",
                                 "hidden_rows", "hidden_dtype", "tokens_len", "tokens_dtype",
                                 "inputs_shape"])
def test_t3_step_rejects_before_launch(bad):
    mod = pkg.load()
    s, m, t = unopened(mod), model(mod), good()
    z = lambda *sh, dt=torch.float32: torch.zeros(sh, dtype=dt)
    kw = dict(tokens=t["tok"])
    if bad == "layers":
        t["k"] = t["v"] = z(2, NL + 1, NH, NCTX, 64)
    elif bad == "heads":
        t["k"] = t["v"] = z(2, NL, NH * 2, NCTX, 64)
    elif bad == "head_dim":
        t["k"] = t["v"] = z(2, NL, NH, NCTX, 128)
    elif bad == "v_shape":
        t["v"] = z(2, NL, NH, NCTX + 1, 64)
    elif bad == "dtype":
        t["k"] = t["k"].double()
    elif bad == "noncontig":
        t["k"] = z(2, NL, NH, 64, NCTX).transpose(-1, -2)
    elif bad == "hidden_rows":
        t["h"] = z(3, NE)
    elif bad == "hidden_dtype":
        t["h"] = t["h"].half()
    elif bad == "tokens_len":
        kw["tokens"] = z(3, dt=torch.int32)
    elif bad == "tokens_dtype":
        kw["tokens"] = z(2, dt=torch.int64)
    elif bad == "inputs_shape":
        kw = dict(inputs=z(2, NE + 1))
    with pytest.raises(ValueError):
        s.t3_step(m, t["pos"], t["k"], t["v"], t["h"], **kw)


def test_t3_prefill_rejects_before_launch():
    mod = pkg.load()
    s, m = unopened(mod), model(mod)
    t = good(rows=5, slots=2)
    slots = torch.zeros(5, dtype=torch.int32)
    inp = torch.zeros((5, NE))
    # a good call gets past the checks (and then fails on the unopened handle)
    with pytest.raises(AttributeError):
        s.t3_prefill(m, slots, t["pos"], t["k"], t["v"], t["h"], inputs=inp, stream=0)
    with pytest.raises(ValueError):  # positions of another row count
        s.t3_prefill(m, slots, torch.zeros(4, dtype=torch.int32), t["k"], t["v"], t["h"],
                     inputs=inp)
    with pytest.raises(ValueError):  # a cache of another layer count
        k = torch.zeros((2, NL - 1, NH, NCTX, 64))
        s.t3_prefill(m, slots, t["pos"], k, k, t["h"], inputs=inp)
    with pytest.raises(ValueError):  # hidden rows for the slots, not the rows
        s.t3_prefill(m, slots, t["pos"], t["k"], t["v"], torch.zeros((2, NE)), inputs=inp)


def test_t3_step_good_arguments_reach_the_library():
    mod = pkg.load()
    s, m, t = unopened(mod), model(mod), good()
    with pytest.raises(AttributeError):  # past the checks: the missing handle
        s.t3_step(m, t["pos"], t["k"], t["v"], t["h"], tokens=t["tok"], stream=0)
