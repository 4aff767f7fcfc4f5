"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on the
same seeded inputs and the same uniforms.

Every case prints its name before touching the GPU.  Sizes are those of the
measured configurations where the oracle finishes in seconds.
"""
import math
import zlib
import os

import numpy as np
import pytest

import debug_lib as D
import oracle_lib as O
import parity
import pkg

pytestmark = pytest.mark.gpu

F32 = np.float32


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


@pytest.fixture(scope="module")
def cbx(torch_cuda):
    # The small-launch rule (calls of at most 512 row-steps run the workgroup
    # kernel at full capacity) is off here, so that each test's launch takes
    # the kernel its survivor bound names; test_latency_rule_* cover the rule.
    mod = pkg.load()
    s = mod.Sampler(device=0, max_vocab=32768, max_history=4096)
    s.set_latency_rows(0)
    yield mod, s
    s.close()


@pytest.fixture(scope="module")
def cbx_default(torch_cuda):
    mod = pkg.load()
    s = mod.Sampler(device=0, max_vocab=32768, max_history=4096)
    yield mod, s
    s.close()


def oparams(d):
    return O.OParams(d["top_k"], d["top_p"], d["temp"], d["repeat_penalty"], d["min_p"],
                     d["cfg_weight"])


def oracle_rows(logits, plist, u, history=None, hist_len=None, uncond=None, allowed=None,
                force_stop=None, stop=0, want_probs=True):
    n = logits.shape[0]
    toks = np.zeros(n, np.int32)
    infos = np.zeros(n, np.uint32)
    probs = np.zeros(logits.shape, np.float32) if want_probs else None
    for r in range(n):
        pr = r % len(plist)
        h = [] if history is None else history[pr][: hist_len[pr]]
        res = O.sample_row(logits[r], h, oparams(plist[pr]), u[r],
                           uncond=None if uncond is None else uncond[r],
                           allowed=None if allowed is None else allowed[pr],
                           force_stop=bool(force_stop[r]) if force_stop is not None else False,
                           stop_token=stop, want_probs=want_probs)
        toks[r], infos[r] = res[0], res[1]
        if want_probs:
            probs[r] = res[2]
    return toks, infos, probs


def gpu_batch(cbx, torch, logits, plist, u=None, history=None, hist_len=None, uncond=None,
              allowed=None, force_stop=None, stop=0, n_steps=1, want_probs=True, **kw):
    mod, s = cbx
    dev = "cuda"
    lg = torch.from_numpy(np.ascontiguousarray(logits)).to(dev)
    n = logits.shape[0]
    w = pkg.workloads()
    prm = torch.from_numpy(w.pack_params(plist)).to(dev)
    tok = torch.full((n,), -7, dtype=torch.int32, device=dev)
    info = torch.zeros(n, dtype=torch.int32, device=dev)
    probs = torch.full(logits.shape, -1.0, dtype=torch.float32, device=dev) if want_probs else None
    args = dict(n_steps=n_steps, info=info, probs=probs, stop_token=stop)
    if u is not None:
        args["uniforms"] = torch.from_numpy(np.ascontiguousarray(u, np.float64)).to(dev)
    if history is not None:
        args["history"] = torch.from_numpy(np.ascontiguousarray(history, np.int32)).to(dev)
        args["history_len"] = torch.from_numpy(np.ascontiguousarray(hist_len, np.int32)).to(dev)
    if uncond is not None:
        args["logits_uncond"] = torch.from_numpy(np.ascontiguousarray(uncond)).to(dev)
    if allowed is not None:
        args["allowed"] = torch.from_numpy(np.ascontiguousarray(allowed, np.uint32).view(np.int32)).to(dev)
    if force_stop is not None:
        args["force_stop"] = torch.from_numpy(np.ascontiguousarray(force_stop, np.uint8)).to(dev)
    args.update(kw)
    s.sample_batch(lg, prm, tok, **args)
    torch.cuda.synchronize()
    return (tok.cpu().numpy(), info.cpu().numpy().view(np.uint32),
            None if probs is None else probs.cpu().numpy())


# --------------------------------------------------------------------------


def test_device_expf_exhaustive(cbx, torch_cuda):
    """The device exponential equals host libm expf for every binary32 input
    the sampler can produce (all x <= 0 down to -104), checked in chunks."""
    torch = torch_cuda
    mod, s = cbx
    lo, hi = 0x80000000, 0xC2D00001
    chunk = 1 << 27
    bad = 0
    start = lo
    while start < hi:
        n = min(chunk, hi - start)
        say(f"expf chunk 0x{start:08x} +{n}")
        bits = torch.arange(n, dtype=torch.int64, device="cuda") + start
        x = (bits - (1 << 32) * (bits >= 2**31).long()).to(torch.int32).view(torch.float32)
        out = torch.empty_like(x)
        D.expf(x, out)
        host = out.cpu().numpy()
        bad += O.lib().cbx_oracle_expf_mismatch(start, n, host.ctypes.data, 16)
        start += n
    assert bad == 0


def test_device_running_sum_scan(cbx, torch_cuda):
    # The workgroup kernel's running sums (wave_run_sum: binade segments with
    # the threshold search in the same pass, sweep chains for short runs, the
    # early stop on sorted terms) against numpy's left-to-right float32
    # accumulation, bit for bit, and the threshold index of the top-p search;
    # 1 to 8192 terms per case.
    import seqsum_cases
    torch = torch_cuda
    mod, s = cbx
    t, off, thr, want_sum, want_hit, desc = seqsum_cases.make_cases(4000, 11, max_n=8192,
                                                                    with_order=True)
    say(f"running sums: {len(off) - 1} cases, {t.size} terms")
    sums = torch.zeros(len(off) - 1, dtype=torch.float32, device="cuda")
    hits = torch.full((len(off) - 1,), -9, dtype=torch.int32, device="cuda")
    D.runsum(torch.from_numpy(t).cuda(), torch.from_numpy(off).cuda(),
             torch.from_numpy(thr).cuda(), torch.from_numpy(desc).cuda(), sums, hits)
    torch.cuda.synchronize()
    got_sum = sums.cpu().numpy()
    got_hit = hits.cpu().numpy()
    bad = np.nonzero(got_sum.view(np.uint32) != want_sum.view(np.uint32))[0]
    assert bad.size == 0, (bad[:5], got_sum[bad[:5]], want_sum[bad[:5]])
    has_thr = thr > 0
    assert np.array_equal(got_hit[has_thr], want_hit[has_thr])
    assert np.array_equal(got_hit[~has_thr], np.full((~has_thr).sum(), -1, np.int32))
    # every run length, both orders and long lists were exercised
    n = np.diff(off)
    assert (n <= 64).sum() > 10 and ((n > 1088) & (desc == 1)).sum() > 100


def test_device_running_sum_short_lists(cbx, torch_cuda):
    # The workgroup kernel's running sums over 1 to 64 terms (one term per
    # lane): sweep chains for at most 8 lanes, binade segments (with the
    # threshold search in the same pass) above that, against numpy's
    # left-to-right float32 accumulation, bit for bit.
    import seqsum_cases
    torch = torch_cuda
    mod, s = cbx
    t, off, thr, want_sum, want_hit, desc = seqsum_cases.make_cases(3000, 29, max_n=64,
                                                                    with_order=True)
    sums = torch.zeros(len(off) - 1, dtype=torch.float32, device="cuda")
    hits = torch.full((len(off) - 1,), -9, dtype=torch.int32, device="cuda")
    D.runsum(torch.from_numpy(t).cuda(), torch.from_numpy(off).cuda(),
             torch.from_numpy(thr).cuda(), torch.from_numpy(desc).cuda(), sums, hits)
    torch.cuda.synchronize()
    got_sum = sums.cpu().numpy()
    got_hit = hits.cpu().numpy()
    bad = np.nonzero(got_sum.view(np.uint32) != want_sum.view(np.uint32))[0]
    assert bad.size == 0, (bad[:5], got_sum[bad[:5]], want_sum[bad[:5]])
    has_thr = thr > 0
    assert np.array_equal(got_hit[has_thr], want_hit[has_thr])
    n = np.diff(off)
    assert (n <= 8).sum() > 100 and ((n > 8) & has_thr).sum() > 300 and ((n > 8) & (desc == 1)).sum() > 1000


def test_device_chain_sums(cbx, torch_cuda):
    # The one-wave kernel's running sums (sweep chains, binade segments for
    # long per-lane runs) against numpy's left-to-right float32 accumulation,
    # bit for bit, and the first index reaching the threshold.
    import seqsum_cases
    torch = torch_cuda
    mod, s = cbx
    t, off, thr, want_sum, want_hit = seqsum_cases.make_cases(8000, 12)
    n = np.diff(off)
    keep = n <= 1088
    # the cases that fit the one-wave layout, repacked
    parts = [t[off[c]:off[c + 1]] for c in np.nonzero(keep)[0]]
    t2 = np.concatenate(parts).astype(np.float32)
    off2 = np.concatenate([[0], np.cumsum([len(x) for x in parts])]).astype(np.int32)
    thr2, want_sum, want_hit = thr[keep], want_sum[keep], want_hit[keep]
    say(f"chain sums: {len(parts)} cases, {t2.size} terms")
    sums = torch.zeros(len(parts), dtype=torch.float32, device="cuda")
    hits = torch.full((len(parts),), -9, dtype=torch.int32, device="cuda")
    D.chainsum(torch.from_numpy(t2).cuda(), torch.from_numpy(off2).cuda(),
                     torch.from_numpy(thr2).cuda(), sums, hits)
    torch.cuda.synchronize()
    got_sum, got_hit = sums.cpu().numpy(), hits.cpu().numpy()
    has_thr = thr2 > 0
    bad = np.nonzero(got_sum[~has_thr].view(np.uint32) != want_sum[~has_thr].view(np.uint32))[0]
    assert bad.size == 0, (bad[:5], got_sum[~has_thr][bad[:5]], want_sum[~has_thr][bad[:5]])
    assert np.array_equal(got_hit[has_thr], want_hit[has_thr])
    # long runs (segments) were exercised
    assert np.sum(np.diff(off2) > 64 * 5) > 100


def test_device_philox_matches_oracle(cbx, torch_cuda):
    torch = torch_cuda
    mod, s = cbx
    say("philox uniforms")
    n = 4096
    sids = np.arange(n, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)
    for seed, step in ((0, 0), (42, 17), (0xDEADBEEFCAFEF00D, 2**40 + 3)):
        out = torch.empty(n, dtype=torch.float64, device="cuda")
        D.philox(seed, torch.from_numpy(sids.view(np.int64)).cuda(), step, n, out)
        got = out.cpu().numpy()
        want = np.array([O.philox_uniform(seed, int(sids[i]), step) for i in range(n)])
        assert np.array_equal(got, want)


def test_single_stream_as_is(cbx, torch_cuda):
    """500 steps, V=6563, k=1000 p=0.95 T=0.8 pen=1.2, min_p=0 (the reference's
    own knobs): uniforms from the reference's mt19937 front end."""
    w = pkg.workloads()
    d = w.single_stream(steps=500, min_p=0.0)
    say("single_stream min_p=0 batch of 500 steps")
    u = O.mt_canonical(42, 500)
    hist = np.tile(d["history"], (1, 1))
    hl = np.array([d["history"].size], np.int32)
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["logits"], [d["params"]], u, hist, hl, n_steps=500,
                           max_survivors=1000)
    tr, ir, pr = oracle_rows(d["logits"], [d["params"]], u, hist, hl)
    parity.compare("single_stream_as_is", tg, ig, tr, ir, u, pg, pr)


def test_single_stream_min_p(cbx, torch_cuda):
    w = pkg.workloads()
    d = w.single_stream(steps=500, min_p=0.05, seed=0x5EED11)
    say("single_stream min_p=0.05")
    u = O.mt_canonical(7, 500)
    hist = d["history"][None, :]
    hl = np.array([d["history"].size], np.int32)
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["logits"], [d["params"]], u, hist, hl, n_steps=500)
    tr, ir, pr = oracle_rows(d["logits"], [d["params"]], u, hist, hl)
    parity.compare("single_stream_min_p", tg, ig, tr, ir, u, pg, pr)


def test_engine_loop_mt19937_row_api(cbx, torch_cuda):
    """The engine's loop (chatterbox_engine.cpp:338-353): one mt19937(seed),
    history growing by each token; the GPU row API fed the uniforms the
    reference's std::discrete_distribution consumed."""
    mod, s = cbx
    w = pkg.workloads()
    d = w.single_stream(steps=200, min_p=0.0, seed=0x5EED12)
    p = d["params"]
    say("engine loop, row API, 200 steps")
    toks, us = O.run_mt19937(d["logits"], np.array([], np.int32), oparams(p), seed=42)
    hist = []
    for t in range(200):
        tok, info = s.sample_row(d["logits"][t], hist, p, us[t])
        assert tok == toks[t], t
        hist.append(tok)


def test_cfg_pair_growing_history(cbx, torch_cuda):
    """CFG pair, V=8194, 1000 steps with the history growing by each sampled
    id: the oracle's id sequence defines every step's history, and one launch
    checks all 1000 steps."""
    w = pkg.workloads()
    d = w.cfg_pair(steps=1000)
    steps = d["cond"].shape[0]
    u = O.mt_canonical(1234, steps)
    say("cfg_pair oracle sequence")
    seq = []
    ref_t, ref_i = np.zeros(steps, np.int32), np.zeros(steps, np.uint32)
    ref_p = np.zeros(d["cond"].shape, np.float32)
    for t in range(steps):
        tok, info, probs, _ = O.sample_row(d["cond"][t], seq, oparams(d["params"]), u[t],
                                           uncond=d["uncond"][t], want_probs=True)
        ref_t[t], ref_i[t], ref_p[t] = tok, info, probs
        seq.append(tok)
    hist = np.zeros((steps, steps), np.int32)
    for t in range(steps):
        hist[t, :t] = seq[:t]
    hl = np.arange(steps, dtype=np.int32)
    say("cfg_pair gpu (1000 rows, one per step)")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["cond"], [d["params"]] * steps, u, hist, hl,
                           uncond=d["uncond"])
    parity.compare("cfg_pair", tg, ig, ref_t, ref_i, u, pg, ref_p)


def test_batched_streams(cbx, torch_cuda):
    """B=256, V=6563, per-row temperature and top-k, 4 independent steps."""
    w = pkg.workloads()
    d = w.batched_streams(B=256, steps=4)
    n = d["logits"].shape[0]
    u = O.mt_canonical(99, n)
    say("batched_streams B=256 x 4 steps")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["logits"], d["params"], u, d["history"],
                           d["hist_len"], n_steps=4, max_survivors=1000)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"])
    parity.compare("batched_streams", tg, ig, tr, ir, u, pg, pr)


@pytest.mark.parametrize("V", [3000, 4000, 5000, 7000, 8300])
def test_batched_streams_vocab(cbx, torch_cuda, V):
    """The batched workload at vocabularies of each one-wave kernel class
    (padding in several vectors per lane, or in the last one only)."""
    w = pkg.workloads()
    d = w.batched_streams(B=256, steps=1, seed=0x5EED40 + V, V=V)
    u = O.mt_canonical(41 + V, 256)
    say(f"batched_streams V={V}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["logits"], d["params"], u, d["history"],
                           d["hist_len"], max_survivors=1000)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"])
    parity.compare(f"batched_streams_{V}", tg, ig, tr, ir, u, pg, pr)


@pytest.mark.parametrize("max_survivors", [0, 1000])
def test_batched_streams_philox(cbx, torch_cuda, max_survivors):
    """Device Philox draws keyed (seed, stream, step) equal the oracle fed the
    oracle's Philox uniforms, on the workgroup kernel (no survivor bound) and
    the one-wave kernel (at most 1000 survivors)."""
    w = pkg.workloads()
    d = w.batched_streams(B=256, steps=2, seed=0x5EED33)
    n = d["logits"].shape[0]
    seed, step0 = 0xC0FFEE, 1000
    u = np.array([O.philox_uniform(seed, r % 256, step0 + r // 256) for r in range(n)])
    say(f"batched_streams philox max_survivors={max_survivors}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["logits"], d["params"], None, d["history"],
                           d["hist_len"], n_steps=2, draw_mode=1, seed=seed, step0=step0,
                           max_survivors=max_survivors)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"])
    parity.compare("batched_streams_philox", tg, ig, tr, ir, u, pg, pr)


def test_timed_path_retry_stream_ids(cbx, torch_cuda):
    """The benchmark's kernel and draw: B=256 streams, 16 steps in one launch,
    at most 1000 survivors (the one-wave kernel), Philox draws keyed by the
    retry policy's stream ids cbx_retry_stream_id(s, a) for attempts 0..3
    (ids up to 3 * 2^56 + 255): every token equals the oracle fed the oracle's
    Philox uniform for that (seed, stream id, step)."""
    torch = torch_cuda
    mod, s = cbx
    w = pkg.workloads()
    B, S = 256, 16
    d = w.batched_streams(B=B, steps=S, seed=0x5EED34)
    n = d["logits"].shape[0]
    sids = np.array([mod.retry_stream_id(r, r % 4) for r in range(B)], np.uint64)
    assert sids.max() >= 3 << 56
    seed, step0 = 0x5EED_F00D, 77
    u = np.array([O.philox_uniform(seed, int(sids[r % B]), step0 + r // B) for r in range(n)])
    say(f"timed path: B={B} x {S} steps, max_survivors=1000, retry stream ids")
    tg, ig, pg = gpu_batch(cbx, torch, d["logits"], d["params"], None, d["history"],
                           d["hist_len"], n_steps=S, draw_mode=1, seed=seed, step0=step0,
                           max_survivors=1000,
                           stream_ids=torch.from_numpy(sids.view(np.int64)).cuda())
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"])
    parity.compare("timed_path_retry_ids", tg, ig, tr, ir, u, pg, pr)
    # the same rows keyed by attempt 0 (the plain stream index) draw differently
    u0 = np.array([O.philox_uniform(seed, r % B, step0 + r // B) for r in range(n)])
    assert np.count_nonzero(u0 != u) == n - n // 4


def test_masked_stress(cbx, torch_cuda):
    """B=1024, V=32768, 20% allowed bitmask, forced stop rows, k=50, p=0.9,
    min_p=0.02, pen=1.3, history 512."""
    w = pkg.workloads()
    d = w.masked_stress()
    u = O.mt_canonical(5, d["B"])
    say("masked_stress B=1024 V=32768")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["logits"], d["params"], u, d["history"],
                           d["hist_len"], allowed=d["allowed"], force_stop=d["force_stop"],
                           stop=d["stop"], max_survivors=50)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"],
                             allowed=d["allowed"], force_stop=d["force_stop"], stop=d["stop"])
    parity.compare("masked_stress", tg, ig, tr, ir, u, pg, pr)
    assert np.all(tg[d["force_stop"] == 1] == d["stop"])


@pytest.mark.parametrize("V", [8449, 12000, 20000, 32768])
def test_chunked_one_wave(cbx, torch_cuda, V):
    """Vocabularies past the register-resident one-wave kernel (V > 8448),
    launches of more than 512 rows and a survivor bound of at most 1024: the
    one-wave kernel reading each row once in chunks, its top-k threshold
    raised as it reads.  Masked rows (allowed bitmask, forced stop), min-p and
    penalty; then batched streams with top_k 50 / 250 / 1000 (the 1000 rows
    overflow its list and take the redo pass), planted rows of tied scores
    at and above the threshold, an all-masked row, and a NaN row (redo; NaN
    is outside the reference's contract: the row is flagged and returns an id
    in range, and the other rows keep parity)."""
    w = pkg.workloads()
    d = w.masked_stress(B=768, V=V, seed=0x5EED9 + V)
    u = O.mt_canonical(23 + V, d["B"])
    say(f"chunked one-wave: masked B=768 V={V}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["logits"], d["params"], u, d["history"],
                           d["hist_len"], allowed=d["allowed"], force_stop=d["force_stop"],
                           stop=d["stop"], max_survivors=50)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"],
                             allowed=d["allowed"], force_stop=d["force_stop"], stop=d["stop"])
    parity.compare(f"chunked_masked_{V}", tg, ig, tr, ir, u, pg, pr)
    d = w.batched_streams(B=256, steps=3, seed=0x5EEDA + V, V=V)
    x = d["logits"]
    rng = np.random.default_rng(V)
    for r in range(0, x.shape[0], 37):  # 70 equal scores above the rest
        x[r, rng.choice(V, size=70, replace=False)] = 13.0
    for r in range(5, x.shape[0], 41):  # 40 equal scores at the threshold's rank
        x[r, rng.choice(V, size=40, replace=False)] = 9.0
        x[r, rng.choice(V, size=30, replace=False)] = 10.0
    x[7, :] = -np.inf  # nothing to sample
    x[9, 100] = np.nan
    n = x.shape[0]
    u = O.mt_canonical(29 + V, n)
    say(f"chunked one-wave: batched streams 256 x 3, V={V}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, d["params"], u, d["history"], d["hist_len"],
                           n_steps=3, max_survivors=1000)
    tr, ir, pr = oracle_rows(x, d["params"], u, d["history"], d["hist_len"])
    assert ig[9] & parity.INFO_NONFINITE and 0 <= tg[9] < V, (ig[9], tg[9])
    ok = np.arange(n) != 9
    parity.compare(f"chunked_batched_{V}", tg[ok], ig[ok], tr[ok], ir[ok], u[ok], pg[ok], pr[ok])


@pytest.mark.parametrize("V", [12000, 32768])
def test_chunked_one_wave_large_launch(cbx, torch_cuda, V):
    """Chunked rows in a launch of more than 2048 row-steps (256 streams x 9
    steps): one wave per row, where the smaller launches above split each
    row's chunks over two waves.  top_k 50 / 250 / 1000, planted ties above
    and at the threshold, an all-masked row."""
    w = pkg.workloads()
    d = w.batched_streams(B=256, steps=9, seed=0x5EEDB + V, V=V)
    x = d["logits"]
    rng = np.random.default_rng(V + 1)
    for r in range(0, x.shape[0], 53):
        x[r, rng.choice(V, size=70, replace=False)] = 13.0
    for r in range(11, x.shape[0], 59):
        x[r, rng.choice(V, size=40, replace=False)] = 9.0
        x[r, rng.choice(V, size=30, replace=False)] = 10.0
    x[3, :] = -np.inf
    n = x.shape[0]
    assert n > 2048
    u = O.mt_canonical(31 + V, n)
    say(f"chunked one-wave, large launch: 256 x 9, V={V}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, d["params"], u, d["history"], d["hist_len"],
                           n_steps=9, max_survivors=1000)
    tr, ir, pr = oracle_rows(x, d["params"], u, d["history"], d["hist_len"])
    parity.compare(f"chunked_large_{V}", tg, ig, tr, ir, u, pg, pr)


@pytest.mark.parametrize("V", [6563, 8194, 3000])
def test_masked_one_wave(cbx, torch_cuda, V):
    """Allowed bitmask, forced stop, min-p and penalty at vocabularies the
    one-wave kernel takes (survivor capacity 1024)."""
    w = pkg.workloads()
    d = w.masked_stress(B=256, V=V, seed=0x5EED5 + V)
    u = O.mt_canonical(11 + V, d["B"])
    say(f"masked one-wave B=256 V={V}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["logits"], d["params"], u, d["history"],
                           d["hist_len"], allowed=d["allowed"], force_stop=d["force_stop"],
                           stop=d["stop"], max_survivors=1024)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"],
                             allowed=d["allowed"], force_stop=d["force_stop"], stop=d["stop"])
    parity.compare(f"masked_one_wave_{V}", tg, ig, tr, ir, u, pg, pr)


def test_cfg_pair_one_wave(cbx, torch_cuda):
    """CFG combine on the one-wave kernel: V=8194 cond/uncond rows with top-k
    1000 (so the survivors fit its list), fixed history."""
    w = pkg.workloads()
    d = w.cfg_pair(steps=256, seed=0x5EED22)
    p = dict(d["params"])
    p["top_k"] = 1000
    rng = np.random.default_rng(3)
    hist = rng.integers(0, 8194, size=(1, 700)).astype(np.int32)
    hl = np.array([700], np.int32)
    u = O.mt_canonical(77, 256)
    say("cfg_pair one-wave 256 steps")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, d["cond"], [p], u, hist, hl, n_steps=256,
                           uncond=d["uncond"], max_survivors=1024)
    tr, ir, pr = oracle_rows(d["cond"], [p], u, hist, hl, uncond=d["uncond"])
    parity.compare("cfg_pair_one_wave", tg, ig, tr, ir, u, pg, pr)


EDGE_CASES = [
    # name, V, params, logits builder, u
    ("all_masked", 64, dict(top_k=10, top_p=0.9, temp=0.8, repeat_penalty=1.2),
     lambda V, r: np.full(V, -np.inf, F32), 0.5),
    ("greedy", 300, dict(top_k=0, top_p=1.0, temp=0.0, repeat_penalty=1.0),
     lambda V, r: np.where(np.arange(V) % 7 == 3, F32(5), F32(1)).astype(F32), 0.5),
    ("greedy_filters", 300, dict(top_k=20, top_p=0.5, temp=-1.0, repeat_penalty=1.5),
     lambda V, r: (r.standard_normal(V) * 3).astype(F32), 0.9),
    ("u_zero", 500, dict(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.2),
     lambda V, r: (r.standard_normal(V) * 3).astype(F32), 0.0),
    ("u_top", 500, dict(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.2),
     lambda V, r: (r.standard_normal(V) * 3).astype(F32), math.nextafter(1.0, 0.0)),
    ("last_id_forced", 4, dict(top_k=0, top_p=1.0, temp=1.0, repeat_penalty=1.0),
     lambda V, r: np.array([0, 0, 0, -np.inf], F32), math.nextafter(1.0, 0.0)),
    ("v1", 1, dict(top_k=0, top_p=0.5, temp=0.8, repeat_penalty=1.2),
     lambda V, r: np.array([3.0], F32), 0.5),
    ("v2", 2, dict(top_k=1, top_p=0.9, temp=0.8, repeat_penalty=1.2),
     lambda V, r: np.array([1.0, 2.0], F32), 0.5),
    ("topk_ties_large", 200, dict(top_k=3, top_p=1.0, temp=1.0, repeat_penalty=1.0),
     lambda V, r: np.concatenate([[9, 5, 5, 5, 5], np.zeros(V - 5)]).astype(F32), 0.7),
    ("topk_ties_small", 200, dict(top_k=3, top_p=1.0, temp=1.0, repeat_penalty=1.0),
     lambda V, r: np.concatenate([[0.5, 1e-4, 1e-4, 1e-4, 1e-4], np.full(V - 5, -1)]).astype(F32),
     0.7),
    ("topp_zero", 300, dict(top_k=0, top_p=0.0, temp=0.8, repeat_penalty=1.2),
     lambda V, r: (r.standard_normal(V) * 3).astype(F32), 0.3),
    ("topp_equal_scores", 64, dict(top_k=0, top_p=0.5, temp=1.0, repeat_penalty=1.0),
     lambda V, r: np.full(V, 2.5, F32), 0.3),
    ("topk_off_full_sort", 6563, dict(top_k=0, top_p=0.95, temp=0.8, repeat_penalty=1.2),
     lambda V, r: (r.standard_normal(V) * 3).astype(F32), 0.61),
    ("topk_eq_V_minus_1", 777, dict(top_k=776, top_p=0.99, temp=1.3, repeat_penalty=0.8),
     lambda V, r: (r.standard_normal(V) * 2).astype(F32), 0.42),
    ("neg_scores_penalty", 900, dict(top_k=100, top_p=0.95, temp=0.8, repeat_penalty=1.7),
     lambda V, r: (r.standard_normal(V) - 20).astype(F32), 0.77),
    ("subnormal_probs", 400, dict(top_k=0, top_p=1.0, temp=1.0, repeat_penalty=1.0),
     lambda V, r: np.concatenate([[0.0], np.full(V - 1, -95.0)]).astype(F32), 0.999),
    ("huge_spread", 2048, dict(top_k=0, top_p=0.999, temp=0.5, repeat_penalty=1.0),
     lambda V, r: (r.standard_normal(V) * 40).astype(F32), 0.5),
    # skewed rows: one spike far above the rest (a single score above the
    # midrange)
    ("topk_spike_refloor", 6563, dict(top_k=50, top_p=0.9, temp=0.9, repeat_penalty=1.2),
     lambda V, r: np.concatenate([[60.0], r.standard_normal(V - 1)]).astype(F32), 0.45),
    # exactly k + 1 scores in the upper half of the range
    ("topk_floor_edge", 2000, dict(top_k=100, top_p=0.95, temp=1.0, repeat_penalty=1.1),
     lambda V, r: np.concatenate([r.uniform(5.0, 6.0, 101), r.uniform(-6.0, -5.0, V - 101)
                                  ]).astype(F32), 0.52),
    # the k-th score ties with the midrange itself (0.0), 60 times
    ("topk_floor_tie", 1500, dict(top_k=50, top_p=0.9, temp=1.0, repeat_penalty=1.3),
     lambda V, r: np.concatenate([[4.0, -4.0], r.uniform(0.5, 3.5, 30), np.zeros(60),
                                  r.uniform(-3.9, -0.1, V - 92)]).astype(F32), 0.66),
    # finite scores whose pairwise products overflow binary32
    ("huge_scores", 6563, dict(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.2),
     lambda V, r: (r.standard_normal(V) * 1e19).astype(F32), 0.4),
    # -inf logits among finite ones (10% of the ids)
    ("some_neg_inf", 6563, dict(top_k=250, top_p=0.9, temp=1.1, repeat_penalty=1.2),
     lambda V, r: np.where(r.random(V) < 0.1, -np.inf, r.standard_normal(V) * 3).astype(F32), 0.6),
    # the one-wave top-k histogram starts at the mean of ids 0..255: here that
    # mean (100.004) is above every score but one, so fewer than k + 1 scores
    # are binned and the full-range pass decides
    ("topk_mean_above_rank", 6563, dict(top_k=1000, top_p=0.9, temp=1.0, repeat_penalty=1.2),
     lambda V, r: np.concatenate([np.full(255, 100.0), [101.0],
                                  r.standard_normal(V - 256)]).astype(F32), 0.3),
    # ... and here (mean 3.906) the 201st largest score, 3.85 held 300 times,
    # lies within the two bins below the mean, whose counts are partial
    ("topk_rank_below_mean_bins", 6563, dict(top_k=200, top_p=0.9, temp=1.0, repeat_penalty=1.2),
     lambda V, r: np.concatenate([np.full(10, 100.0), np.zeros(246), np.full(300, 3.85),
                                  -5.0 - r.random(V - 556)]).astype(F32), 0.7),
    # every finite score equal (the top-k threshold in closed form): more than
    # k of them at 4.0 (the nudge is a no-op: nothing survives), more than k
    # at 1e-4 (the nudge keeps them all), one finite id (a forced-stop row),
    # fewer than k finite ids, more than k finite ids among -inf
    ("all_equal_topk_large", 500, dict(top_k=10, top_p=0.9, temp=1.0, repeat_penalty=1.2),
     lambda V, r: np.full(V, 4.0, F32), 0.5),
    ("all_equal_topk_small", 500, dict(top_k=10, top_p=0.9, temp=1.0, repeat_penalty=1.2),
     lambda V, r: np.full(V, 1e-4, F32), 0.5),
    ("one_finite_topk", 6563, dict(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.3),
     lambda V, r: np.where(np.arange(V) == 6562, F32(3.0), F32(-np.inf)).astype(F32), 0.5),
    ("few_finite_equal", 6563, dict(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.3),
     lambda V, r: np.where(np.arange(V) % 219 == 5, F32(2.0), F32(-np.inf)).astype(F32), 0.5),
    ("many_finite_equal", 6563, dict(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.3),
     lambda V, r: np.where(np.arange(V) % 64 == 5, F32(2.0), F32(-np.inf)).astype(F32), 0.5),
    # 150 equal survivors in one value bin: the sort falls back to the bitonic network
    ("crowded_bin", 600, dict(top_k=500, top_p=0.9, temp=1.0, repeat_penalty=1.2),
     lambda V, r: np.concatenate([np.full(150, 3.0), np.full(200, 2.0), [10.0],
                                  r.standard_normal(V - 351) - 3.0]).astype(F32), 0.37),
]


@pytest.mark.parametrize("case", EDGE_CASES, ids=[c[0] for c in EDGE_CASES])
def test_edge_cases(cbx, torch_cuda, case):
    name, V, p, build, u = case
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    pd = dict(min_p=0.0, cfg_weight=0.0)
    pd.update(p)
    x = build(V, rng)[None, :]
    hist = rng.integers(-5, V + 5, size=(1, 64)).astype(np.int32)
    hl = np.array([64], np.int32)
    uu = np.array([u])
    say(f"edge {name} V={V}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, [pd], uu, hist, hl)
    tr, ir, pr = oracle_rows(x, [pd], uu, hist, hl)
    parity.compare(f"edge_{name}", tg, ig, tr, ir, uu, pg, pr)
    # the single-row host API gives the batched path's answer (and the
    # oracle's, unless the row is a counted top-p tie)
    mod, s = cbx
    tok, info = s.sample_row(x[0], hist[0], pd, u)
    # (the diagnostic TOPP_SORTED bit depends on the kernel each call ran)
    diag = parity.INFO_TOPP_SORTED
    assert tok == tg[0] and (info & ~diag) == (int(ig[0]) & ~diag)
    assert tok == tr[0]


# cases whose survivors after top-k fit the one-wave kernel's list
WAVE_EDGE = [c for c in EDGE_CASES if c[1] <= 1024 or 0 < c[2].get("top_k", 0) <= 1024]


@pytest.mark.parametrize("case", WAVE_EDGE, ids=[c[0] for c in WAVE_EDGE])
def test_edge_cases_one_wave(cbx, torch_cuda, case):
    """The same rows through the one-wave kernel (survivor capacity 1024)."""
    name, V, p, build, u = case
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    pd = dict(min_p=0.0, cfg_weight=0.0)
    pd.update(p)
    x = build(V, rng)[None, :]
    hist = rng.integers(-5, V + 5, size=(1, 64)).astype(np.int32)
    hl = np.array([64], np.int32)
    uu = np.array([u])
    say(f"edge one-wave {name} V={V}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, [pd], uu, hist, hl, max_survivors=1024)
    tr, ir, pr = oracle_rows(x, [pd], uu, hist, hl)
    parity.compare(f"edge_wave_{name}", tg, ig, tr, ir, uu, pg, pr)


@pytest.mark.parametrize("max_survivors", [0, 1024])
def test_nonfinite_rows_flagged(cbx, torch_cuda, max_survivors):
    """NaN or +inf logits are outside the reference's contract: such rows are
    flagged CBX_INFO_NONFINITE and still return an id in range (or -1 on
    overflow); rows of the same batch without them keep parity."""
    V = 6563
    rng = np.random.default_rng(41)
    x = (rng.standard_normal((6, V)) * 3).astype(F32)
    x[0, 17] = np.nan
    x[1, 3000] = np.inf
    x[2, 5] = np.nan
    x[2, 6] = -np.inf
    x[3, :] = np.nan
    # rows 4 and 5 stay finite
    plist = [dict(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.2, min_p=0.0, cfg_weight=0.0)] * 6
    u = rng.random(6)
    hist = rng.integers(0, V, size=(6, 64)).astype(np.int32)
    hl = np.full(6, 64, np.int32)
    say(f"nonfinite rows max_survivors={max_survivors}")
    tg, ig, _ = gpu_batch(cbx, torch_cuda, x, plist, u, hist, hl, max_survivors=max_survivors)
    for r in range(4):
        assert ig[r] & parity.INFO_NONFINITE, (r, ig[r])
        assert -1 <= tg[r] < V
    assert not np.any(ig[4:] & parity.INFO_NONFINITE)
    tr, ir, _ = oracle_rows(x[4:], plist[4:], u[4:], hist[4:], hl[4:])
    assert list(tg[4:]) == list(tr)


def test_row_api_extensions(cbx, torch_cuda):
    """cbx_sample_row_ex with CFG, mask, forced stop and probabilities out."""
    mod, s = cbx
    w = pkg.workloads()
    rng = np.random.default_rng(3)
    V = 8194
    say("row api extensions")
    for t in range(30):
        c = (rng.standard_normal(V) * 3).astype(F32)
        un = (c + rng.standard_normal(V)).astype(F32)
        bits = rng.random((1, V)) < 0.5
        al = w.pack_bitmask(bits)[0]
        p = dict(top_k=int(rng.integers(0, 2000)), top_p=float(rng.uniform(0.5, 1.0)),
                 temp=float(rng.uniform(0.3, 1.5)), repeat_penalty=1.2,
                 min_p=float(rng.choice([0.0, 0.05])), cfg_weight=0.5)
        h = rng.integers(0, V, size=100)
        u = float(rng.random())
        fs = bool(t % 10 == 9)
        tok, info, probs = s.sample_row(c, h, p, u, logits_uncond=un, allowed=al, force_stop=fs,
                                        stop_token=V - 2, want_probs=True)
        tr, ir, pr, _ = O.sample_row(c, h, oparams(p), u, uncond=un, allowed=al, force_stop=fs,
                                     stop_token=V - 2, want_probs=True)
        parity.compare(f"row_ext_{t}", [tok], [info], [tr], [ir], [u], probs[None], pr[None])


def test_golden_fixtures(cbx, torch_cuda):
    path = os.path.join(os.path.dirname(__file__), "golden", "sampler_cases.npz")
    g = np.load(path)
    n = g["logits"].shape[0]
    say(f"golden fixtures ({n} rows)")
    plist = [dict(zip(("top_k", "top_p", "temp", "repeat_penalty", "min_p", "cfg_weight"),
                      (int(r[0]),) + tuple(float(v) for v in r[1:]))) for r in g["params"]]
    tg, ig, pg = gpu_batch(cbx, torch_cuda, g["logits"], plist, g["u"], g["history"],
                           g["hist_len"], allowed=g["allowed"])
    parity.compare("golden", tg, ig, g["tokens"], g["info"], g["u"], pg, g["probs"])


def plateau_rows(rng, n, V, plateau, level=8.0):
    """Rows whose top-p cutoff falls inside a run of equal scores: three
    spikes (10, 9.5, 9), `plateau` ids at `level` scattered over the row and
    the rest far below.  At T = 1 and p = 0.5 the cumulative mass crosses p
    among the plateau's ids."""
    x = (rng.standard_normal((n, V)) - 6.0).astype(F32)
    for r in range(n):
        ids = rng.choice(V, size=plateau + 3, replace=False)
        x[r, ids[:3]] = [10.0, 9.5, 9.0]
        x[r, ids[3:]] = level
    return x


TIE_CASES = [
    # name, V, top_k, plateau, max_survivors (kernel)
    ("one_wave", 6563, 1000, 200, 1024),      # one-wave kernel, list of 1000
    ("one_wave_small", 500, 100, 60, 1024),
    ("wg_fast", 6563, 1000, 300, 0),          # workgroup kernel, register list
    ("wg_general", 8194, 0, 3000, 0),         # workgroup kernel, sorted scores (8194
                                              # survivors): one lane replays the sort
    ("wg_general_wave", 3000, 0, 1000, 0),    # 3000 survivors: the wavefront replay
]


@pytest.mark.parametrize("case", TIE_CASES, ids=[c[0] for c in TIE_CASES])
def test_topp_tie_rows(cbx, torch_cuda, case):
    """Equal scores straddle the top-p cutoff in every row: the kept ids are
    the ones the reference's std::sort puts first, so tokens and
    probabilities equal the oracle's (which runs std::sort itself)."""
    name, V, k, plateau, ms = case
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    n = 4 if name.startswith("wg_general") else 32
    x = plateau_rows(rng, n, V, plateau)
    plist = [dict(top_k=k, top_p=0.5, temp=1.0, repeat_penalty=1.3, min_p=0.0,
                  cfg_weight=0.0)] * n
    hist = rng.integers(0, V, size=(n, 200)).astype(np.int32)
    hl = np.full(n, 200, np.int32)
    u = rng.random(n)
    say(f"top-p tie rows {name}: n={n} V={V} k={k} plateau={plateau} max_survivors={ms}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, plist, u, hist, hl, max_survivors=ms)
    tr, ir, pr = oracle_rows(x, plist, u, hist, hl)
    assert np.count_nonzero(ir & parity.INFO_TOPP_TIE) == n  # every row is a tie row
    parity.compare(f"topp_tie_{name}", tg, ig, tr, ir, u, pg, pr)


def test_batch_overflow_rows_redone(cbx, torch_cuda):
    """cbx_sample_batch at max_survivors=1000 (the one-wave kernel, 1024
    survivors) on a batch where some rows keep far more ids: a top-k
    threshold tied at 1e-5 (the -1e-10f nudge keeps every tie), and rows with
    top-k off.  Those rows are sampled again at the vocabulary's capacity in
    the same call: every token is the oracle's, no row reports overflow."""
    V, n = 6563, 12
    rng = np.random.default_rng(0x0F10)
    x = (rng.standard_normal((n, V)) * 3).astype(F32)
    plist = []
    for r in range(n):
        kind = r % 3
        if kind == 0:      # 40 ids above 1e-5, 1500 tied at it: k=100 keeps 1540
            x[r] = -1.0 - rng.random(V).astype(F32)
            ids = rng.choice(V, size=1540, replace=False)
            x[r, ids[:40]] = rng.uniform(1e-3, 2e-3, 40).astype(F32)
            x[r, ids[40:]] = F32(1e-5)
            plist.append(dict(top_k=100, top_p=0.999, temp=1.0, repeat_penalty=1.2, min_p=0.0,
                              cfg_weight=0.0))
        elif kind == 1:    # top-k off: every id survives
            plist.append(dict(top_k=0, top_p=0.95, temp=0.8, repeat_penalty=1.2, min_p=0.0,
                              cfg_weight=0.0))
        else:              # an ordinary row
            plist.append(dict(top_k=250, top_p=0.9, temp=0.9, repeat_penalty=1.2, min_p=0.0,
                              cfg_weight=0.0))
    hist = rng.integers(0, V, size=(n, 100)).astype(np.int32)
    hl = np.full(n, 100, np.int32)
    u = rng.random(n)
    say("batch overflow rows redone at full capacity (one-wave launch)")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, plist, u, hist, hl, max_survivors=1000)
    tr, ir, pr = oracle_rows(x, plist, u, hist, hl)
    assert np.all(tg >= 0)
    parity.compare("batch_overflow_redo", tg, ig, tr, ir, u, pg, pr)


def test_batch_overflow_past_redo_list(cbx, torch_cuda):
    """More overflowing row-steps in one call than the redo list holds (4096):
    4200 rows with top-k off at max_survivors=64.  Exactly 4096 of them are
    sampled again (which ones depends on the order the rows finish), each the
    oracle's token; the other 104 keep token -1 and CBX_INFO_OVERFLOW."""
    V, n, redo_len = 600, 4200, 4096
    rng = np.random.default_rng(0x4200)
    x = (rng.standard_normal((n, V)) * 2).astype(F32)
    plist = [dict(top_k=0, top_p=0.9, temp=0.9, repeat_penalty=1.2, min_p=0.0,
                  cfg_weight=0.0)] * n
    hist = rng.integers(0, V, size=(n, 32)).astype(np.int32)
    hl = np.full(n, 32, np.int32)
    u = rng.random(n)
    say(f"batch overflow past the redo list: n={n} V={V} max_survivors=64")
    tg, ig, _ = gpu_batch(cbx, torch_cuda, x, plist, u, hist, hl, max_survivors=64,
                          want_probs=False)
    done = tg >= 0
    assert np.count_nonzero(done) == redo_len
    assert np.all(tg[~done] == -1)
    assert np.all(ig[~done] & parity.INFO_OVERFLOW)
    assert not np.any(ig[done] & parity.INFO_OVERFLOW)
    tr, ir, _ = oracle_rows(x, plist, u, hist, hl, want_probs=False)
    parity.compare("batch_overflow_past_redo", tg[done], ig[done], tr[done], ir[done], u[done])


@pytest.mark.parametrize("max_survivors", [0, 50])
def test_topk_off_full_vocab_32768(cbx, torch_cuda, max_survivors):
    """top_k = 0 at V = 32768: all 32768 ids survive top-k, so top-p sorts the
    whole row (the workgroup kernel's score sort at capacity 32768).  With a
    hint of 50 the first launch cannot hold them and the second pass does."""
    V, n = 32768, 3
    rng = np.random.default_rng(0x32768 + max_survivors)
    x = (rng.standard_normal((n, V)) * 3).astype(F32)
    plist = [dict(top_k=0, top_p=p, temp=0.8, repeat_penalty=1.3, min_p=0.0, cfg_weight=0.0)
             for p in (0.95, 0.5, 0.999)]
    hist = rng.integers(0, V, size=(n, 512)).astype(np.int32)
    hl = np.full(n, 512, np.int32)
    u = rng.random(n)
    say(f"top-k off V=32768 max_survivors={max_survivors}")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, plist, u, hist, hl, max_survivors=max_survivors)
    tr, ir, pr = oracle_rows(x, plist, u, hist, hl)
    parity.compare(f"topk_off_32768_{max_survivors}", tg, ig, tr, ir, u, pg, pr)


def _sorted_prefix(x_row, k, T):
    """Survivors of top-k (k + 1-th largest cut) in descending order and the
    binary64 prefix ratios of their exp terms (a planning aid for the rows
    below; the oracle decides every result)."""
    s = (x_row * F32(1.0 / T)).astype(F32) if T != 1.0 else x_row
    thr = np.sort(s)[::-1][k]
    surv = np.sort(s[s > thr])[::-1]
    e = np.exp(surv.astype(np.float64) - surv[0])
    return surv, np.cumsum(e) / e.sum()


def test_topp_value_bin_paths(cbx, torch_cuda):
    """The one-wave kernel decides top-p on value bins (no sort) when the
    bound of the reference's float sums certifies the cutoff, and otherwise
    sorts and sums exactly (CBX_INFO_TOPP_SORTED).  Rows built for each
    route, all against the oracle: ordinary rows (mostly certified); the
    cutoff inside a bin of 30 close scores (ranked in the bin, certified);
    top_p set to a cumulative value itself (within the bound: sorted); the
    cutoff inside a bin of 100 close scores (more than one row of the bin:
    sorted); equal scores across the cutoff (tie rows: sorted, std::sort's
    order replayed)."""
    rng = np.random.default_rng(0x70BB)
    V = 6563
    rows, plist, kind = [], [], []

    def add(x, k, p, T, tag):
        rows.append(x.astype(F32))
        plist.append(dict(top_k=k, top_p=float(F32(p)), temp=T, repeat_penalty=1.2, min_p=0.0,
                          cfg_weight=0.0))
        kind.append(tag)

    for r in range(96):
        add(rng.standard_normal(V) * 3, [50, 250, 1000][r % 3], 0.9, 0.8, "plain")
    for r in range(32):  # the cutoff inside one bin of 30 close scores
        x = rng.standard_normal(V) - 8.0
        ids = rng.choice(V, size=31, replace=False)
        x[ids[0]] = 10.0
        x[ids[1:]] = 4.0 + rng.permutation(30) * 1e-4
        surv, y = _sorted_prefix(x.astype(F32), 40, 1.0)
        m = int(rng.integers(6, 24))
        add(x, 40, (y[m - 1] + y[m]) / 2, 1.0, "bin30")
    for r in range(32):  # top_p equal to a cumulative value: within the bound
        x = rng.standard_normal(V) * 3
        surv, y = _sorted_prefix(x.astype(F32), 250, 1.0)
        add(x, 250, y[int(rng.integers(20, 200))], 1.0, "on_bound")
    for r in range(16):  # the cutoff inside one bin of 100 close scores
        x = rng.standard_normal(V) - 8.0
        ids = rng.choice(V, size=101, replace=False)
        x[ids[0]] = 10.0
        x[ids[1:]] = 4.0 + rng.permutation(100) * 1e-5
        surv, y = _sorted_prefix(x.astype(F32), 120, 1.0)
        add(x, 120, (y[40] + y[41]) / 2, 1.0, "bin100")
    tie = plateau_rows(rng, 16, V, 200)
    for r in range(16):
        add(tie[r], 1000, 0.5, 1.0, "tie")
    x = np.stack(rows)
    n = x.shape[0]
    kind = np.array(kind)
    hist = rng.integers(0, V, size=(n, 300)).astype(np.int32)
    hl = rng.integers(0, 301, size=n).astype(np.int32)
    u = rng.random(n)
    say(f"top-p value-bin paths: {n} rows, one-wave kernel")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, plist, u, hist, hl, max_survivors=1024)
    tr, ir, pr = oracle_rows(x, plist, u, hist, hl)
    parity.compare("topp_value_bins", tg, ig, tr, ir, u, pg, pr)
    srt = (ig & parity.INFO_TOPP_SORTED) != 0
    frac = {k: float(srt[kind == k].mean()) for k in np.unique(kind)}
    say(f"  sorted fraction per kind: {frac}")
    assert frac["plain"] < 0.25 and frac["bin30"] == 0.0
    assert frac["on_bound"] == 1.0 and frac["bin100"] == 1.0 and frac["tie"] == 1.0
    assert np.all((ir[kind == "tie"] & parity.INFO_TOPP_TIE) != 0)


def test_topp_open_cut_workgroup_kernel(cbx_default, torch_cuda):
    """The workgroup kernel's top-p cut where its certificate cannot decide:
    top_p equal to a cumulative value, or one float step either side of it,
    so the exact sum of the q's runs over the prefix the bound leaves open
    (and over the whole list should that prefix fall short).  A launch of
    96 rows takes the workgroup kernel under the small-launch rule; the same
    rows with the rule off take the one-wave kernel; both against the
    oracle and against each other."""
    mod, s = cbx_default
    rng = np.random.default_rng(0x0C07)
    V = 6563
    rows, plist = [], []
    for r in range(96):
        k = [250, 1000, 1000][r % 3]
        x = (rng.standard_normal(V) * [3.0, 1.0, 0.5][r % 3]).astype(F32)
        surv, y = _sorted_prefix(x, k, 1.0)
        m = int(rng.integers(5, max(6, int(np.searchsorted(y, 0.999)))))  # top_p < 1 in float
        p = F32(y[m])
        p = [p, np.nextafter(p, F32(1)), np.nextafter(p, F32(0))][(r // 3) % 3]
        rows.append(x)
        plist.append(dict(top_k=k, top_p=float(p), temp=1.0, repeat_penalty=1.2, min_p=0.0,
                          cfg_weight=0.0))
    x = np.stack(rows)
    n = x.shape[0]
    hist = rng.integers(0, V, size=(n, 300)).astype(np.int32)
    hl = rng.integers(0, 301, size=n).astype(np.int32)
    u = rng.random(n)
    say(f"top-p open cuts: {n} rows, workgroup kernel (small-launch rule on)")
    on = gpu_batch(cbx_default, torch_cuda, x, plist, u, hist, hl)
    say("top-p open cuts: same rows, one-wave kernel (rule off)")
    s.set_latency_rows(0)
    try:
        off = gpu_batch(cbx_default, torch_cuda, x, plist, u, hist, hl, max_survivors=1024)
    finally:
        s.set_latency_rows(512)
    tr, ir, pr = oracle_rows(x, plist, u, hist, hl)
    parity.compare("topp_open_cut_wg", on[0], on[1], tr, ir, u, on[2], pr)
    parity.compare("topp_open_cut_wave", off[0], off[1], tr, ir, u, off[2], pr)
    diag = np.uint32(parity.INFO_TOPP_SORTED)  # the one-wave kernel's diagnostic bit
    assert np.array_equal(on[0], off[0]) and np.array_equal(on[1] & ~diag, off[1] & ~diag)
    assert np.count_nonzero(off[1] & diag) > n // 2  # the bound straddles top_p


def test_topp_tie_full_vocab_32768(cbx, torch_cuda):
    """Equal scores across the top-p cutoff with every id of V = 32768
    surviving: the replay of std::sort runs on 16-bit score ranks."""
    V, n = 32768, 2
    rng = np.random.default_rng(0x77E)
    x = plateau_rows(rng, n, V, 5000)
    plist = [dict(top_k=0, top_p=0.5, temp=1.0, repeat_penalty=1.3, min_p=0.0,
                  cfg_weight=0.0)] * n
    hist = rng.integers(0, V, size=(n, 300)).astype(np.int32)
    hl = np.full(n, 300, np.int32)
    u = rng.random(n)
    say("top-p tie rows, V=32768, top-k off")
    tg, ig, pg = gpu_batch(cbx, torch_cuda, x, plist, u, hist, hl)
    tr, ir, pr = oracle_rows(x, plist, u, hist, hl)
    assert np.all(ir & parity.INFO_TOPP_TIE)
    parity.compare("topp_tie_32768", tg, ig, tr, ir, u, pg, pr)


# ---------------------------------------------- the small-launch rule (default)

def test_latency_rule_batched_streams(cbx_default, torch_cuda):
    """Default handle: B=256 streams x 2 steps (512 row-steps) with the
    survivor bound 1000 run on the workgroup kernel at full capacity; Philox
    draws; every token, flag and probability the oracle's."""
    w = pkg.workloads()
    d = w.batched_streams(B=256, steps=2, seed=0x5EED35)
    n = d["logits"].shape[0]
    seed, step0 = 0xFACE, 3
    u = np.array([O.philox_uniform(seed, r % 256, step0 + r // 256) for r in range(n)])
    say("latency rule: batched streams 256 x 2, max_survivors=1000")
    tg, ig, pg = gpu_batch(cbx_default, torch_cuda, d["logits"], d["params"], None, d["history"],
                           d["hist_len"], n_steps=2, draw_mode=1, seed=seed, step0=step0,
                           max_survivors=1000)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"])
    parity.compare("latency_rule_batched", tg, ig, tr, ir, u, pg, pr)


@pytest.mark.parametrize("V", [6563, 8194, 3000])
def test_latency_rule_masked(cbx_default, torch_cuda, V):
    """Default handle: masked rows with forced stops, min-p and penalty, 256
    rows at survivor bound 1024 (full capacity under the rule)."""
    w = pkg.workloads()
    d = w.masked_stress(B=256, V=V, seed=0x5EED7 + V)
    u = O.mt_canonical(13 + V, d["B"])
    say(f"latency rule: masked B=256 V={V}")
    tg, ig, pg = gpu_batch(cbx_default, torch_cuda, d["logits"], d["params"], u, d["history"],
                           d["hist_len"], allowed=d["allowed"], force_stop=d["force_stop"],
                           stop=d["stop"], max_survivors=1024)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"],
                             allowed=d["allowed"], force_stop=d["force_stop"], stop=d["stop"])
    parity.compare(f"latency_rule_masked_{V}", tg, ig, tr, ir, u, pg, pr)


@pytest.mark.parametrize("V", [1000, 4096, 6656, 8192, 12000, 16384, 20000, 32768])
def test_latency_rule_vocab_classes(cbx_default, torch_cuda, V):
    """Default handle: 64 streams x 2 steps with the survivor bound 1000 at
    every vocabulary class of the workgroup kernel (512 lanes x 8, 13, 16;
    1024 lanes x 16, 32), at and past each class's end."""
    w = pkg.workloads()
    d = w.batched_streams(B=64, steps=2, seed=0x5EED50 + V, V=V)
    n = d["logits"].shape[0]
    u = O.mt_canonical(51 + V, n)
    say(f"latency rule: batched streams 64 x 2, V={V}")
    tg, ig, pg = gpu_batch(cbx_default, torch_cuda, d["logits"], d["params"], u, d["history"],
                           d["hist_len"], n_steps=2, max_survivors=1000)
    tr, ir, pr = oracle_rows(d["logits"], d["params"], u, d["history"], d["hist_len"])
    parity.compare(f"latency_rule_V{V}", tg, ig, tr, ir, u, pg, pr)


def test_latency_rule_same_results_either_way(cbx_default, torch_cuda):
    """The rule changes the kernel, not the result: a CFG batch of 128 rows
    with top-p ties and tiny top-k ties sampled with the rule on and off is
    identical bit for bit (tokens, flags, probabilities) and the oracle's."""
    torch = torch_cuda
    mod, s = cbx_default
    rng = np.random.default_rng(0x1A7E)
    V, n = 6563, 128
    x = (rng.standard_normal((n, V)) * 3).astype(np.float32)
    un = (x + rng.standard_normal((n, V))).astype(np.float32)
    plist = []
    for r in range(n):
        if r % 3 == 0:  # equal scores across the top-p cutoff
            ids = rng.choice(V, size=120, replace=False)
            x[r, ids[:2]] = [14.0, 13.0]
            x[r, ids[2:]] = 11.0
            un[r, ids] = x[r, ids]
        plist.append(dict(top_k=1000 if r % 3 == 0 else [50, 250][r % 2],
                          top_p=0.6 if r % 3 == 0 else 0.95,
                          temp=0.8, repeat_penalty=1.2, min_p=0.02, cfg_weight=0.5))
    hist = rng.integers(0, V, size=(n, 300)).astype(np.int32)
    hl = rng.integers(0, 301, size=n).astype(np.int32)
    u = rng.random(n)
    say("latency rule on/off: CFG 128 rows")
    on = gpu_batch(cbx_default, torch, x, plist, u, hist, hl, uncond=un, max_survivors=1000)
    s.set_latency_rows(0)
    try:
        off = gpu_batch(cbx_default, torch, x, plist, u, hist, hl, uncond=un, max_survivors=1000)
    finally:
        s.set_latency_rows(512)
    diag = np.uint32(parity.INFO_TOPP_SORTED)  # the one-wave kernel's diagnostic bit
    assert np.array_equal(on[0], off[0]) and np.array_equal(on[1] & ~diag, off[1] & ~diag)
    assert np.array_equal(on[2].view(np.uint32), off[2].view(np.uint32))
    tr, ir, pr = oracle_rows(x, plist, u, hist, hl, uncond=un)
    parity.compare("latency_rule_on_off", on[0], on[1], tr, ir, u, on[2], pr)
    assert np.count_nonzero(on[1] & parity.INFO_TOPP_TIE) > 10
