"""cbx_sample_batch_static (the redo list in the library's file-scope device
array, no allocation) against cbx_sample_batch (the handle's list): the same
tokens, flags and probabilities, bit for bit, on two calls in a row -- the
second smaller -- whose batches hold rows that need the redo pass (more
survivors than max_survivors), rows whose top-p cutoff falls inside equal
scores, and ordinary rows; and the tokens are the oracle's."""
import numpy as np
import pytest

import oracle_lib as O
import parity
import pkg

pytestmark = pytest.mark.gpu

F32 = np.float32


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def mixed_rows(rng, n, V):
    x = (rng.standard_normal((n, V)) * 3).astype(F32)
    plist = []
    for r in range(n):
        kind = r % 4
        if kind == 0:  # 40 ids above 1e-5, 1500 tied at it: k = 100 keeps 1540
            x[r] = -1.0 - rng.random(V).astype(F32)
            ids = rng.choice(V, size=1540, replace=False)
            x[r, ids[:40]] = rng.uniform(1e-3, 2e-3, 40).astype(F32)
            x[r, ids[40:]] = F32(1e-5)
            plist.append(dict(top_k=100, top_p=0.999, temp=1.0, repeat_penalty=1.2))
        elif kind == 1:  # top-k off: every id survives
            plist.append(dict(top_k=0, top_p=0.95, temp=0.8, repeat_penalty=1.2))
        elif kind == 2:  # equal scores across the top-p cutoff
            x[r] = (rng.standard_normal(V) - 6.0).astype(F32)
            ids = rng.choice(V, size=203, replace=False)
            x[r, ids[:3]] = [10.0, 9.5, 9.0]
            x[r, ids[3:]] = 8.0
            plist.append(dict(top_k=1000, top_p=0.5, temp=1.0, repeat_penalty=1.3))
        else:
            plist.append(dict(top_k=250, top_p=0.9, temp=0.9, repeat_penalty=1.2))
    for p in plist:
        p.update(min_p=0.0, cfg_weight=0.0)
    return x, plist


def run(mod, s, torch, x, plist, hist, hl, u, static):
    w = pkg.workloads()
    n = x.shape[0]
    tok = torch.full((n,), -7, dtype=torch.int32, device="cuda")
    info = torch.zeros(n, dtype=torch.int32, device="cuda")
    probs = torch.full(x.shape, -1.0, dtype=torch.float32, device="cuda")
    s.sample_batch(torch.from_numpy(x).cuda(), torch.from_numpy(w.pack_params(plist)).cuda(), tok,
                   uniforms=torch.from_numpy(u).cuda(), history=torch.from_numpy(hist).cuda(),
                   history_len=torch.from_numpy(hl).cuda(), info=info, probs=probs,
                   max_survivors=1000, static_scratch=static)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), info.cpu().numpy().view(np.uint32), probs.cpu().numpy()


def test_static_scratch_matches_batch():
    torch = pytest.importorskip("torch")
    assert torch.cuda.is_available()
    mod = pkg.load()
    s = mod.Sampler(device=0, max_vocab=32768, max_history=1024)
    # these calls are small: with the small-launch rule off they keep the
    # survivor bound, so the redo list is used
    s.set_latency_rows(0)
    V = 6563
    rng = np.random.default_rng(0x57A71C)
    for n in (40, 10):  # two calls in a row, the second smaller
        x, plist = mixed_rows(rng, n, V)
        hist = rng.integers(0, V, size=(n, 100)).astype(np.int32)
        hl = np.full(n, 100, np.int32)
        u = rng.random(n)
        say(f"static redo list: {n} rows")
        ts, is_, ps = run(mod, s, torch, x, plist, hist, hl, u, True)
        say(f"handle redo list: {n} rows")
        tb, ib, pb = run(mod, s, torch, x, plist, hist, hl, u, False)
        assert np.array_equal(ts, tb) and np.array_equal(is_, ib)
        assert np.array_equal(ps.view(np.uint32), pb.view(np.uint32))
        assert np.all(ts >= 0)
        # and both are the oracle's
        op = [O.OParams(p["top_k"], p["top_p"], p["temp"], p["repeat_penalty"], 0.0, 0.0)
              for p in plist]
        ref = [O.sample_row(x[r], hist[r], op[r], u[r], want_probs=True) for r in range(n)]
        parity.compare(f"static_{n}", ts, is_, [t[0] for t in ref], [t[1] for t in ref], u, ps,
                       np.stack([t[2] for t in ref]))
    # beyond the list's 4096 rows with a hint below the vocabulary: refused
    big = torch.zeros((4097, 300), dtype=torch.float32, device="cuda")
    prm = torch.from_numpy(pkg.workloads().pack_params(
        [dict(top_k=5, top_p=0.9, temp=1.0, repeat_penalty=1.0, min_p=0.0, cfg_weight=0.0)])).cuda()
    tok = torch.zeros(4097, dtype=torch.int32, device="cuda")
    with pytest.raises(mod.CbxError):
        s.sample_batch(big, prm.repeat(4097), tok, max_survivors=5, static_scratch=True)
    # ... unless the small-launch rule covers the call: then it runs at full
    # capacity (no redo list) and gives the handle call's tokens
    s.set_latency_rows(8192)
    xb = rng.standard_normal((4200, 300)).astype(F32)
    pb = torch.from_numpy(pkg.workloads().pack_params(
        [dict(top_k=50, top_p=0.9, temp=0.9, repeat_penalty=1.0, min_p=0.0,
              cfg_weight=0.0)])).cuda().repeat(4200)
    ub = torch.from_numpy(rng.random(4200)).cuda()
    outs = []
    for static in (True, False):
        say(f"4200 rows under the small-launch rule, static={static}")
        t = torch.full((4200,), -7, dtype=torch.int32, device="cuda")
        s.sample_batch(torch.from_numpy(xb).cuda(), pb, t, uniforms=ub, max_survivors=5,
                       static_scratch=static)
        torch.cuda.synchronize()
        outs.append(t.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]) and np.all(outs[0] >= 0)
    s.close()
