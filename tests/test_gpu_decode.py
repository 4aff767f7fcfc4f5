"""GPU parity of the device-resident decode step (cbx_decode_step,
cbx_head_decode_step) against the engine's decode loop
(src/chatterbox_engine.cpp:337-356) restated on the host with the oracle
sampler.

The T3 step graph is out of this build, so a deterministic stand-in takes its
place on both sides: the logits (or the ln_f rows) of stream r at step t are
row (7 * token_in + 13 * t + 3 * r) mod NB of a fixed bank, token_in being the
id the stream fed back (the start id at step 0).  A stream's result then
depends on every id it sampled before, as in the real loop.  Draws are
Philox keyed (seed, stream r, step t) on the device and the oracle's Philox
uniform of the same key on the host.
"""
import numpy as np
import pytest

import oracle_lib as O
import pkg

pytestmark = pytest.mark.gpu

V, STOP, START = 6563, 6562, 6561  # the Turbo vocabulary; stop and start ids
SEED = 0xDEC0DE


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


@pytest.fixture(scope="module")
def cbx(torch_cuda):
    # launches take the kernel their survivor bound names (no small-launch rule)
    mod = pkg.load()
    s = mod.Sampler(device=0, max_vocab=32768, max_history=4096)
    s.set_latency_rows(0)
    yield mod, s
    s.close()


PLIST = [
    dict(top_k=1000, top_p=0.95, temp=0.8, repeat_penalty=1.2, min_p=0.0, cfg_weight=0.0),
    dict(top_k=50, top_p=0.9, temp=1.0, repeat_penalty=1.5, min_p=0.05, cfg_weight=0.0),
    dict(top_k=250, top_p=0.8, temp=0.7, repeat_penalty=1.1, min_p=0.0, cfg_weight=0.0),
    dict(top_k=1000, top_p=1.0, temp=0.0, repeat_penalty=1.3, min_p=0.0, cfg_weight=0.0),
]


def _bank(rng, nb, v=V):
    """Logit rows: N(0, 2) with five spikes; every 11th row puts the stop id
    (v - 1) 4 above its largest, so streams end at varied steps."""
    b = (rng.standard_normal((nb, v)) * 2.0).astype(np.float32)
    for j in range(nb):
        b[j, rng.integers(0, v - 2, 5)] += 3.0
        if j % 11 == 0:
            b[j, v - 1] = b[j].max() + 4.0
    return b


def _idx(tok_in, t, r, nb):
    return (7 * int(tok_in) + 13 * t + 3 * r) % nb


def engine_loop(r, logits_of, p, max_len, stop=STOP, start=START):
    """chatterbox_engine.cpp:337-356 for stream r: sample on the first
    logits, push, then while fewer than n_predict steps ran: stop on the stop
    id, run the step graph on the last id, sample, push; the trailing stop id
    is dropped.  Returns (generated, ended on stop, tokens per step)."""
    n_predict = max_len - 1
    generated, steps = [], []
    cur = O.sample_row(logits_of(r, start, 0), np.array(generated, np.int32), p,
                       O.philox_uniform(SEED, r, 0))[0]
    generated.append(cur)
    steps.append(cur)
    for i in range(n_predict):
        if cur == stop:
            break
        cur = O.sample_row(logits_of(r, cur, i + 1), np.array(generated, np.int32), p,
                           O.philox_uniform(SEED, r, i + 1))[0]
        generated.append(cur)
        steps.append(cur)
    stopped = generated[-1] == stop
    if stopped:
        generated.pop()
    return generated, stopped, steps


@pytest.mark.parametrize("v", [V, 16000])
def test_decode_loop_matches_engine_loop(cbx, torch_cuda, v):
    """16 streams, up to 40 steps of cbx_decode_step with no host copy between
    steps: each stream's history, length, state, fed-back id and per-step
    tokens equal the engine loop's on the oracle (the 512-lane decode kernel
    at V 6563, the 1024-lane one at V 16000)."""
    torch = torch_cuda
    mod, s = cbx
    B, T, NB, LD = 16, 40, 97, 64
    stop, start = v - 1, v - 2
    rng = np.random.default_rng(0xDEC1)
    bank = _bank(rng, NB, v)
    # every stream ends within the T steps (at most max_len ids, one per step)
    max_len = np.array([[8, 20, 40, 33][r % 4] if r % 5 else 30 for r in range(B)], np.int32)
    max_len[3] = 1  # one id, then the limit
    plist = [PLIST[r % 4] for r in range(B)]
    w = pkg.workloads()
    dbank = torch.from_numpy(bank).cuda()
    prm = torch.from_numpy(w.pack_params(plist)).cuda()
    state = torch.zeros(B, dtype=torch.int32, device="cuda")
    hist = torch.full((B, LD), -9, dtype=torch.int32, device="cuda")
    hlen = torch.zeros(B, dtype=torch.int32, device="cuda")
    nxt = torch.full((B,), start, dtype=torch.int32, device="cuda")
    dmax = torch.from_numpy(max_len).cuda()
    toks = torch.full((T, B), -5, dtype=torch.int32, device="cuda")
    infos = torch.zeros((T, B), dtype=torch.int32, device="cuda")
    rows = torch.arange(B, device="cuda")
    dec = mod.Sampler.decode_state(state, hist, hlen, max_len=dmax, next_token=nxt)
    say(f"decode loop B={B} T={T} V={v}")
    for t in range(T):
        idx = (7 * nxt.long() + 13 * t + 3 * rows) % NB
        lg = dbank[idx]
        s.decode_step(lg, prm, toks[t], dec, info=infos[t], seed=SEED, step0=t,
                      stop_token=stop)
    torch.cuda.synchronize()
    st, hi, hl = state.cpu().numpy(), hist.cpu().numpy(), hlen.cpu().numpy()
    nx, tk, inf = nxt.cpu().numpy(), toks.cpu().numpy(), infos.cpu().numpy()

    def logits_of(r, tok_in, t):
        return bank[_idx(tok_in, t, r, NB)]

    n_stop = 0
    for r in range(B):
        gen, stopped, steps = engine_loop(r, logits_of, O.params(**plist[r]), int(max_len[r]),
                                          stop, start)
        n_stop += stopped
        assert hl[r] == len(gen), (r, hl[r], len(gen))
        assert list(hi[r, :hl[r]]) == gen, r
        assert np.all(hi[r, hl[r]:] == -9), r  # nothing written past the length
        assert st[r] == (mod.CBX_DECODE_STOP if stopped else mod.CBX_DECODE_LIMIT), (r, st[r])
        assert nx[r] == (gen[-1] if gen else start), r
        n = len(steps)
        assert list(tk[:n, r]) == steps, r
        # once ended, a stream is not sampled: stop id, CBX_INFO_ENDED
        assert np.all(tk[n:, r] == stop) and np.all(inf[n:, r] == mod.CBX_INFO_ENDED), r
        assert not np.any(inf[:n, r] & mod.CBX_INFO_ENDED), r
    assert 0 < n_stop < B  # both endings occur


def test_decode_many_streams(cbx, torch_cuda):
    """4200 streams (V 300, top-k off: every id survives) in one decode step,
    with a survivor bound of 64 passed and ignored (a decode step runs at full
    capacity): every stream's token, history, length, state and next id equal
    the engine loop's step on the oracle, from histories already holding 0 to
    5 ids, a third of them one id from their limit."""
    torch = torch_cuda
    mod, s = cbx
    B, Vs, LD = 4200, 300, 16
    rng = np.random.default_rng(0xDEC2)
    lg = rng.standard_normal((B, Vs)).astype(np.float32)
    stop = 7
    lg[::13, stop] += 6.0
    h0 = rng.integers(0, Vs, size=(B, LD)).astype(np.int32)
    hl0 = rng.integers(0, 6, size=B).astype(np.int32)
    h0[np.arange(LD)[None, :] >= hl0[:, None]] = -9
    max_len = np.where(np.arange(B) % 3 == 0, hl0 + 1, LD).astype(np.int32)
    p = dict(top_k=0, top_p=0.9, temp=1.0, repeat_penalty=1.3, min_p=0.0, cfg_weight=0.0)
    w = pkg.workloads()
    prm = torch.from_numpy(w.pack_params([p] * B)).cuda()
    state = torch.zeros(B, dtype=torch.int32, device="cuda")
    hist = torch.from_numpy(h0).cuda()
    hlen = torch.from_numpy(hl0).cuda()
    nxt = torch.full((B,), -3, dtype=torch.int32, device="cuda")
    tok = torch.full((B,), -5, dtype=torch.int32, device="cuda")
    info = torch.zeros(B, dtype=torch.int32, device="cuda")
    dec = mod.Sampler.decode_state(state, hist, hlen, max_len=torch.from_numpy(max_len).cuda(),
                                   next_token=nxt)
    say(f"decode many streams B={B} V={Vs}")
    s.decode_step(torch.from_numpy(lg).cuda(), prm, tok, dec, info=info, seed=SEED, step0=5,
                  stop_token=stop, max_survivors=64)
    torch.cuda.synchronize()
    st, hi, hl = state.cpu().numpy(), hist.cpu().numpy(), hlen.cpu().numpy()
    nx, tk, inf = nxt.cpu().numpy(), tok.cpu().numpy(), info.cpu().numpy()
    assert not np.any(inf & mod.CBX_INFO_OVERFLOW)
    op = O.params(**p)
    n_stop = 0
    for r in range(B):
        want = O.sample_row(lg[r], h0[r, :hl0[r]], op, O.philox_uniform(SEED, r, 5))[0]
        assert tk[r] == want, r
        if want == stop:
            n_stop += 1
            assert st[r] == mod.CBX_DECODE_STOP and hl[r] == hl0[r] and nx[r] == -3, r
        else:
            assert hl[r] == hl0[r] + 1 and hi[r, hl0[r]] == want and nx[r] == want, r
            lim = hl0[r] + 1 if r % 3 == 0 else LD
            assert st[r] == (mod.CBX_DECODE_LIMIT if hl[r] >= lim else mod.CBX_DECODE_RUNNING), r
        assert np.array_equal(hi[r, :hl0[r]], h0[r, :hl0[r]]), r
    assert n_stop > 0


def test_head_decode_loop_matches_engine_loop(cbx, torch_cuda):
    """The fused step: 32 CFG streams (64 ln_f rows, the matrix-core
    projection of a Q4_0 head, V 6563, n_embd 1024), 16 steps of
    cbx_head_decode_step.  Every step's logits are the head's (binary64 head
    within the projection bound) and each stream's ids are the engine loop's
    on the oracle run on the logits the GPU projected."""
    torch = torch_cuda
    mod, s = cbx
    B, T, NB, K, LD = 32, 16, 41, 1024, 32
    rng = np.random.default_rng(0xDEC3)
    wq = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    blocks = O.quantize(wq, O.WTYPE_Q4_0)
    bias = (rng.standard_normal(V) * 0.1).astype(np.float32)
    bias[STOP] = 1.5
    hb = rng.standard_normal((NB, K)).astype(np.float32)
    hbu = (hb + 0.5 * rng.standard_normal(hb.shape)).astype(np.float32)
    plist = [dict(PLIST[r % 4], cfg_weight=0.5) for r in range(B)]
    max_len = np.full(B, T, np.int32)
    w = pkg.workloads()
    dW = torch.from_numpy(blocks.reshape(-1)).cuda()
    db = torch.from_numpy(bias).cuda()
    dhb, dhbu = torch.from_numpy(hb).cuda(), torch.from_numpy(hbu).cuda()
    prm = torch.from_numpy(w.pack_params(plist)).cuda()
    state = torch.zeros(B, dtype=torch.int32, device="cuda")
    hist = torch.full((B, LD), -9, dtype=torch.int32, device="cuda")
    hlen = torch.zeros(B, dtype=torch.int32, device="cuda")
    nxt = torch.full((B,), START, dtype=torch.int32, device="cuda")
    toks = torch.full((T, B), -5, dtype=torch.int32, device="cuda")
    lc = torch.zeros((T, B, V), dtype=torch.float32, device="cuda")
    lu = torch.zeros_like(lc)
    idxs = torch.zeros((T, B), dtype=torch.int64, device="cuda")
    rows = torch.arange(B, device="cuda")
    dec = mod.Sampler.decode_state(state, hist, hlen, max_len=torch.from_numpy(max_len).cuda(),
                                   next_token=nxt)
    say(f"head decode loop Q4_0 B={B} CFG T={T}")
    for t in range(T):
        idxs[t] = (7 * nxt.long() + 13 * t + 3 * rows) % NB
        hc, hu = dhb[idxs[t]], dhbu[idxs[t]]
        head = mod.Sampler.head(dW, O.WTYPE_Q4_0, K, hc, lc[t], bias=db, hidden_uncond=hu,
                                logits_uncond=lu[t])
        s.decode_step(lc[t], prm, toks[t], dec, head=head, seed=SEED, step0=t, stop_token=STOP)
    torch.cuda.synchronize()
    st, hi, hl = state.cpu().numpy(), hist.cpu().numpy(), hlen.cpu().numpy()
    lcn, lun, ix = lc.cpu().numpy(), lu.cpu().numpy(), idxs.cpu().numpy()
    # the projection of two steps' rows is the head's
    for t in (0, T // 2):
        for x, bank in ((lcn[t], hb), (lun[t], hbu)):
            hh = bank[ix[t]]
            ref = O.head_f64(blocks, O.WTYPE_Q4_0, bias, hh, V, K)
            deq = np.abs(O.dequantize(blocks, O.WTYPE_Q4_0, K)).astype(np.float64)
            ah = np.abs(hh).astype(np.float64)
            tol = 1e-5 * (ah @ deq.T) + 2.0 ** -39 * ah.max(1)[:, None] * deq.sum(1) + 1e-6
            assert np.all(np.abs(x - ref) <= tol)

    # the engine loop on the GPU's logits: valid while the ids agree, since
    # the step graph's rows follow from them
    n_stop = 0
    for r in range(B):
        def logits_of(rr, tok_in, t, r=r):
            assert ix[t, r] == _idx(tok_in, t, r, NB), (r, t)
            return lcn[t, r]

        p = O.params(**plist[r])
        gen, stopped, steps = [], False, []
        cur_in = START
        for t in range(T):
            lgt = logits_of(r, cur_in, t)
            cur = O.sample_row(lgt, np.array(gen, np.int32), p, O.philox_uniform(SEED, r, t),
                               uncond=lun[t, r])[0]
            steps.append(cur)
            if cur == STOP:
                stopped = True
                break
            gen.append(cur)
            cur_in = cur
            if len(gen) >= max_len[r]:
                break
        n_stop += stopped
        assert hl[r] == len(gen) and list(hi[r, :hl[r]]) == gen, r
        assert st[r] == (mod.CBX_DECODE_STOP if stopped else mod.CBX_DECODE_LIMIT), (r, st[r])
    assert n_stop > 0


def test_decode_rejects_bad_arguments(cbx, torch_cuda):
    torch = torch_cuda
    mod, s = cbx
    w = pkg.workloads()
    prm = torch.from_numpy(w.pack_params([PLIST[0]] * 2)).cuda()
    lg = torch.zeros((2, 2, 64), dtype=torch.float32, device="cuda")
    tok = torch.zeros(4, dtype=torch.int32, device="cuda")
    state = torch.zeros(2, dtype=torch.int32, device="cuda")
    hist = torch.zeros((2, 8), dtype=torch.int32, device="cuda")
    hlen = torch.zeros(2, dtype=torch.int32, device="cuda")
    dec = mod.Sampler.decode_state(state, hist, hlen)
    with pytest.raises(mod.CbxError):  # a decode step samples one step
        s.decode_step(lg, prm, tok, dec, n_steps=2)
    bad = mod.Sampler.decode_state(state, hist, hlen)
    bad.state = None
    with pytest.raises(mod.CbxError):
        s.decode_step(lg[0], prm, tok[:2], bad)
    bad = mod.Sampler.decode_state(state, hist[:, :0], hlen)  # ld_history 0
    with pytest.raises(mod.CbxError):
        s.decode_step(lg[0], prm, tok[:2], bad)
    torch.cuda.synchronize()
