"""GPU parity of the T3 transformer's decode step (cbx_t3_step,
chatterbox.cpp_amd/csrc/cbx_t3.hip) against the binary64 oracle
(oracle/cbx_t3_oracle.py), on the Turbo shape (24 layers, n_embd 1024, 16
heads of 64) with random weights in each matrix format, and the whole
batched decode loop on the device: T3 step, fused head, sampler, ids fed
back.

Tolerance on ln_f's output rows: |gpu - ref| <= 5e-5 + 5e-5 |ref|.  The GPU
computes in binary32 (the reference's own dtype: fp32 activations, fp32 KV
cache, main.cpp:419-424) through 24 layers of products over 1024 to 4096
terms, each layer's residual re-normalized; the oracle in binary64 with the
same dequantized weights.  Values are O(1) after ln_f; the largest error
measured over every case here is 3.2e-6 (about 50 binary32 ulps of 1), and
the bound allows 15 times that.  A wrong head offset, a missing residual or
a cache row written at the wrong position moves rows by O(1).
"""
import numpy as np
import pytest

import oracle_lib as O
import pkg
from oracle import cbx_t3_oracle as T3

pytestmark = pytest.mark.gpu

N_CTX_LONG = 4096  # caches of the reference's context scale (n_ctx 8196, n_predict 1000)

N_LAYER, N, H, N_POS, V = 24, 1024, 16, 64, 6563
TOL_ABS, TOL_REL = 5e-5, 5e-5


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


@pytest.fixture(scope="module")
def cbx(torch_cuda):
    mod = pkg.load()
    s = mod.Sampler(device=0, max_vocab=32768, max_history=4096)
    yield mod, s
    s.close()


_MODELS = {}


def model(torch, mod, wtype, n_pos=N_POS):
    """Random Turbo-shaped weights in `wtype` (matrices N(0, 0.02)): the
    device model and the oracle's binary64 copy of the same values.  A model
    with more positions (n_pos) shares the layers of the N_POS one and takes
    its own wpe rows."""
    if n_pos != N_POS:
        key = (wtype, n_pos)
        if key not in _MODELS:
            dm0, rm0 = model(torch, mod, wtype)
            rng = np.random.default_rng(0x7301 + n_pos)
            wpe = (rng.standard_normal((n_pos, N)) * 0.1).astype(np.float32)
            t = lambda a: torch.from_numpy(a).cuda()
            layers = dm0._keep[1]
            _, _, _, emb, gf, bf = dm0._keep
            dm = mod.Sampler.t3_model(layers, t(wpe), emb, gf, bf, wtype=wtype, n_head=H)
            rm = T3.Model(rm0.layers, wpe, rm0.speech_emb, rm0.ln_f_g, rm0.ln_f_b, 1e-5, H)
            _MODELS[key] = (dm, rm)
        return _MODELS[key]
    if wtype in _MODELS:
        return _MODELS[wtype]
    rng = np.random.default_rng(0x7300 + wtype)
    vec = lambda k, base=0.0, sd=0.1: (base + rng.standard_normal(k) * sd).astype(np.float32)
    dev_layers, ref_layers = [], []
    for _ in range(N_LAYER):
        d, r = {}, {}
        for key, (o, i) in (("attn_w", (3 * N, N)), ("attn_proj_w", (N, N)), ("fc_w", (4 * N, N)),
                            ("fc_proj_w", (N, 4 * N))):
            w = (rng.standard_normal((o, i)) * 0.02).astype(np.float32)
            blocks = O.quantize(w, wtype)
            d[key] = torch.from_numpy(blocks.reshape(-1)).cuda()
            r[key] = O.dequantize(blocks, wtype, i)
        for key, k, base, sd in (("ln_1_g", N, 1.0, 0.1), ("ln_1_b", N, 0.0, 0.1),
                                 ("attn_b", 3 * N, 0.0, 0.02), ("attn_proj_b", N, 0.0, 0.02),
                                 ("ln_2_g", N, 1.0, 0.1), ("ln_2_b", N, 0.0, 0.1),
                                 ("fc_b", 4 * N, 0.0, 0.02), ("fc_proj_b", N, 0.0, 0.02)):
            a = vec(k, base, sd)
            d[key] = torch.from_numpy(a).cuda()
            r[key] = a
        dev_layers.append(d)
        ref_layers.append(r)
    wpe = (rng.standard_normal((N_POS, N)) * 0.1).astype(np.float32)
    emb = (rng.standard_normal((V, N)) * 0.5).astype(np.float32)
    gf, bf = vec(N, 1.0), vec(N)
    t = lambda a: torch.from_numpy(a).cuda()
    dm = mod.Sampler.t3_model(dev_layers, t(wpe), t(emb), t(gf), t(bf), wtype=wtype, n_head=H)
    rm = T3.Model(ref_layers, wpe, emb, gf, bf, 1e-5, H)
    _MODELS[wtype] = (dm, rm)
    return dm, rm


def close(got, want):
    err = np.abs(got.astype(np.float64) - want)
    return np.all(err <= TOL_ABS + TOL_REL * np.abs(want)), float(err.max())


@pytest.mark.parametrize("B", [20, 5, 2, 1])
@pytest.mark.parametrize("wtype", [O.WTYPE_Q4_0, O.WTYPE_Q5_0, O.WTYPE_Q8_0, O.WTYPE_F16])
def test_t3_step_matches_oracle(cbx, torch_cuda, wtype, B):
    """B streams, 4 steps with per-stream ids; in step 2 every third stream
    sits out (state not running), so positions differ afterwards.  Each step's
    ln_f rows, every stream's position and the skipped rows' zeros match the
    oracle.  B = 20 runs the products on the matrix cores, B = 5 on the
    mat-vec; B = 2 and 1 fold the residual adds and norms between a layer's
    products into the mat-vec that consumes them."""
    torch = torch_cuda
    mod, s = cbx
    dm, rm = model(torch, mod, wtype)
    rng = np.random.default_rng(0x7310 + B)
    kd = torch.zeros((B, N_LAYER, H, N_POS, 64), dtype=torch.float32, device="cuda")
    vd = torch.zeros_like(kd)
    kr, vr = T3.new_cache(B, N_LAYER, H, N_POS)
    pos_d = torch.zeros(B, dtype=torch.int32, device="cuda")
    pos_r = np.zeros(B, np.int64)
    hid = torch.zeros((B, N), dtype=torch.float32, device="cuda")
    worst = 0.0
    for t in range(4):
        toks = rng.integers(0, V, B).astype(np.int32)
        state = np.zeros(B, np.int32)
        if t == 2:
            state[::3] = 1
        say(f"t3 step wtype={wtype} B={B} t={t}")
        s.t3_step(dm, pos_d, kd, vd, hid, tokens=torch.from_numpy(toks).cuda(),
                  state=torch.from_numpy(state).cuda())
        torch.cuda.synchronize()
        want = T3.step(rm, toks, pos_r, kr, vr, active=state == 0)
        got = hid.cpu().numpy()
        ok, err = close(got, want)
        worst = max(worst, err)
        assert ok, f"step {t}: max err {err:.3g}"
        assert np.all(got[state != 0] == 0.0)
        assert np.array_equal(pos_d.cpu().numpy(), pos_r)
    say(f"  max |err| {worst:.3g}")


def test_t3_folded_norms_match_separate(cbx, torch_cuda):
    """Two streams (norms folded into the mat-vec products) give bit for bit
    the rows the same two streams give beside a third (separate norm
    kernels): the folded norm repeats the norm kernel's operations in its
    order, and every kernel's row results are independent of the other
    rows.  Step 1 has stream 1 sitting out (its residual carried through)."""
    torch = torch_cuda
    mod, s = cbx
    dm, _ = model(torch, mod, O.WTYPE_Q4_0)
    rng = np.random.default_rng(0x7320)
    outs = {}
    toks = rng.integers(0, V, (3, 3)).astype(np.int32)
    for B in (2, 3):
        kd = torch.zeros((B, N_LAYER, H, N_POS, 64), dtype=torch.float32, device="cuda")
        vd = torch.zeros_like(kd)
        pos = torch.zeros(B, dtype=torch.int32, device="cuda")
        hid = torch.zeros((B, N), dtype=torch.float32, device="cuda")
        rows = []
        for t in range(3):
            state = np.zeros(B, np.int32)
            if t == 1:
                state[1] = 1
            say(f"t3 folded B={B} t={t}")
            s.t3_step(dm, pos, kd, vd, hid, tokens=torch.from_numpy(toks[t, :B].copy()).cuda(),
                      state=torch.from_numpy(state).cuda())
            torch.cuda.synchronize()
            rows.append(hid.cpu().numpy()[:2].copy())
        outs[B] = np.stack(rows)
    assert np.array_equal(outs[2].view(np.uint32), outs[3].view(np.uint32))


def test_t3_inputs_then_tokens(cbx, torch_cuda):
    """Prompt rows fed as embedded inputs (one position per call), then ids:
    the same ln_f rows as the oracle fed the same rows."""
    torch = torch_cuda
    mod, s = cbx
    dm, rm = model(torch, mod, O.WTYPE_Q4_0)
    B = 16
    rng = np.random.default_rng(0x7320)
    kd = torch.zeros((B, N_LAYER, H, N_POS, 64), dtype=torch.float32, device="cuda")
    vd = torch.zeros_like(kd)
    kr, vr = T3.new_cache(B, N_LAYER, H, N_POS)
    pos_d = torch.zeros(B, dtype=torch.int32, device="cuda")
    pos_r = np.zeros(B, np.int64)
    hid = torch.zeros((B, N), dtype=torch.float32, device="cuda")
    for t in range(5):
        say(f"t3 inputs/tokens t={t}")
        if t < 3:
            rows = (rng.standard_normal((B, N)) * 0.5).astype(np.float32)
            s.t3_step(dm, pos_d, kd, vd, hid, inputs=torch.from_numpy(rows).cuda())
            want = T3.step(rm, None, pos_r, kr, vr, inputs=rows)
        else:
            toks = rng.integers(0, V, B).astype(np.int32)
            s.t3_step(dm, pos_d, kd, vd, hid, tokens=torch.from_numpy(toks).cuda())
            want = T3.step(rm, toks, pos_r, kr, vr)
        torch.cuda.synchronize()
        ok, err = close(hid.cpu().numpy(), want)
        assert ok, f"step {t}: max err {err:.3g}"


def test_t3_head_decode_loop(cbx, torch_cuda):
    """The whole decode loop on the device for 16 streams, 8 steps: T3 step
    on the fed-back ids, the fused Q4_0 speech_head and the sampler
    (cbx_head_decode_step), no host copy between steps.  Afterwards, step by
    step: the T3 rows match the oracle fed the same ids, the logits the head
    of those rows, and every id is the oracle sampler's on the GPU's logits
    with the history so far."""
    torch = torch_cuda
    mod, s = cbx
    dm, rm = model(torch, mod, O.WTYPE_Q4_0)
    B, T, LD = 16, 8, 16
    stop, start = -1, V - 2  # no id stops a stream: all 16 run the 8 steps
    rng = np.random.default_rng(0x7330)
    hw = (rng.standard_normal((V, N)) * 0.02).astype(np.float32)
    hblocks = O.quantize(hw, O.WTYPE_Q4_0)
    hbias = (rng.standard_normal(V) * 0.1).astype(np.float32)
    plist = [dict(top_k=1000, top_p=0.95, temp=0.8, repeat_penalty=1.2, min_p=0.0,
                  cfg_weight=0.0)] * B
    w = pkg.workloads()
    prm = torch.from_numpy(w.pack_params(plist)).cuda()
    dW = torch.from_numpy(hblocks.reshape(-1)).cuda()
    db = torch.from_numpy(hbias).cuda()
    kd = torch.zeros((B, N_LAYER, H, N_POS, 64), dtype=torch.float32, device="cuda")
    vd = torch.zeros_like(kd)
    pos_d = torch.zeros(B, dtype=torch.int32, device="cuda")
    state = torch.zeros(B, dtype=torch.int32, device="cuda")
    hist = torch.full((B, LD), -9, dtype=torch.int32, device="cuda")
    hlen = torch.zeros(B, dtype=torch.int32, device="cuda")
    nxt = torch.full((B,), start, dtype=torch.int32, device="cuda")
    hids = torch.zeros((T, B, N), dtype=torch.float32, device="cuda")
    logits = torch.zeros((T, B, V), dtype=torch.float32, device="cuda")
    toks = torch.full((T, B), -5, dtype=torch.int32, device="cuda")
    ins = torch.zeros((T, B), dtype=torch.int32, device="cuda")
    dec = mod.Sampler.decode_state(state, hist, hlen, next_token=nxt)
    say(f"t3 + head decode loop B={B} T={T}")
    for t in range(T):
        ins[t] = nxt
        s.t3_step(dm, pos_d, kd, vd, hids[t], tokens=nxt, state=state)
        head = mod.Sampler.head(dW, O.WTYPE_Q4_0, N, hids[t], logits[t], bias=db)
        s.decode_step(logits[t], prm, toks[t], dec, head=head, seed=0x7331, step0=t,
                      stop_token=stop)
    torch.cuda.synchronize()
    hid_g, lg_g = hids.cpu().numpy(), logits.cpu().numpy()
    tok_g, in_g = toks.cpu().numpy(), ins.cpu().numpy()
    kr, vr = T3.new_cache(B, N_LAYER, H, N_POS)
    pos_r = np.zeros(B, np.int64)
    gen = [[] for _ in range(B)]
    op = O.params(**plist[0])
    hdeq = np.abs(O.dequantize(hblocks, O.WTYPE_Q4_0, N)).astype(np.float64)
    for t in range(T):
        # the ids each stream fed back: its previous token (start at step 0)
        want_in = np.array([gen[r][-1] if gen[r] else start for r in range(B)])
        assert np.array_equal(in_g[t], want_in), t
        want = T3.step(rm, want_in, pos_r, kr, vr)
        ok, err = close(hid_g[t], want)
        assert ok, f"step {t}: T3 rows max err {err:.3g}"
        # the head's bound (tests/test_gpu_head.py): fp32 sums plus the split floor
        ref = O.head_f64(hblocks, O.WTYPE_Q4_0, hbias, hid_g[t], V, N)
        ah = np.abs(hid_g[t]).astype(np.float64)
        tol = 1e-5 * (ah @ hdeq.T) + 2.0 ** -39 * ah.max(1)[:, None] * hdeq.sum(1) + 1e-6
        assert np.all(np.abs(lg_g[t] - ref) <= tol), t
        for r in range(B):
            u = O.philox_uniform(0x7331, r, t)
            tk = O.sample_row(lg_g[t, r], np.array(gen[r], np.int32), op, u)[0]
            assert tok_g[t, r] == tk, (t, r)
            gen[r].append(tk)
    assert np.array_equal(pos_d.cpu().numpy(), np.full(B, T))
    assert np.array_equal(hlen.cpu().numpy(), np.full(B, T))


def test_t3_rejects_bad_arguments(cbx, torch_cuda):
    torch = torch_cuda
    mod, s = cbx
    dm, _ = model(torch, mod, O.WTYPE_Q4_0)
    pos = torch.zeros(2, dtype=torch.int32, device="cuda")
    toks = torch.zeros(2, dtype=torch.int32, device="cuda")
    hid = torch.zeros((2, N), dtype=torch.float32, device="cuda")
    kd = torch.zeros((2, N_LAYER, H, N_POS, 64), dtype=torch.float32, device="cuda")
    big = torch.zeros((2, N_LAYER, H, N_POS + 1, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(mod.CbxError):  # n_ctx above the model's positions
        s.t3_step(dm, pos, big, big, hid, tokens=toks)
    n_head = dm.n_head
    dm.n_head = 8  # 128-wide heads
    k8 = torch.zeros((2, N_LAYER, 8, N_POS, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(mod.CbxError):
        s.t3_step(dm, pos, k8, k8, hid, tokens=toks)
    dm.n_head = n_head
    with pytest.raises(ValueError):  # a cache built for another head count
        s.t3_step(dm, pos, k8, k8, hid, tokens=toks)
    with pytest.raises(mod.CbxError):  # neither ids nor input rows
        s.t3_step(dm, pos, kd, kd, hid)
    torch.cuda.synchronize()


@pytest.mark.parametrize("wtype", [O.WTYPE_Q8_0, O.WTYPE_Q5_0])
@pytest.mark.parametrize("B", [18, 3])
def test_t3_from_gguf(cbx, torch_cuda, tmp_path, B, wtype):
    """A T3 GGUF (2 layers, n_embd 256, Q8_0 or Q5_0 matrices -- the
    converter's --quant q8_0 / q5_0 -- speech_emb F16 as the converter writes
    it) loaded by cbx_gguf_load_t3 into one device buffer: 3 steps of
    cbx_t3_step match the oracle built from the file's values."""
    import test_gguf_t3 as GT
    torch = torch_cuda
    mod, s = cbx
    rng = np.random.default_rng(0x7340 + B + wtype)
    data, vals = GT.make_t3(rng, wtype=wtype)
    path = tmp_path / "t3.gguf"
    path.write_bytes(data)
    say(f"t3 from gguf B={B} wtype={wtype}")
    info, dm = mod.load_t3_gguf(str(path))
    assert (info.n_layer, info.n_embd, info.wtype) == (2, 256, wtype)
    rm = T3.Model(vals["layers"], vals["wpe"], vals["speech_emb"], vals["ln_f_g"],
                  vals["ln_f_b"], 1e-5, 4)
    kd = torch.zeros((B, 2, 4, 32, 64), dtype=torch.float32, device="cuda")
    vd = torch.zeros_like(kd)
    kr, vr = T3.new_cache(B, 2, 4, 32)
    pos_d = torch.zeros(B, dtype=torch.int32, device="cuda")
    pos_r = np.zeros(B, np.int64)
    hid = torch.zeros((B, 256), dtype=torch.float32, device="cuda")
    for t in range(3):
        toks = rng.integers(0, 300, B).astype(np.int32)
        s.t3_step(dm, pos_d, kd, vd, hid, tokens=torch.from_numpy(toks).cuda())
        torch.cuda.synchronize()
        want = T3.step(rm, toks, pos_r, kr, vr)
        ok, err = close(hid.cpu().numpy(), want)
        assert ok, f"step {t}: max err {err:.3g}"


@pytest.mark.parametrize("lens", [(5, 9, 7), (2, 3)])
def test_t3_prefill_then_decode(cbx, torch_cuda, lens):
    """Prompts of several streams in one cbx_t3_prefill call (rows in shuffled
    order, embedded input rows), then two cbx_t3_step decode steps: every
    prompt row's ln_f output matches the oracle stepping each stream through
    its positions one at a time (the causal prompt pass), and the decode
    steps continue from the caches the prefill wrote.  21 rows take the
    matrix cores, 5 the mat-vec."""
    torch = torch_cuda
    mod, s = cbx
    dm, rm = model(torch, mod, O.WTYPE_Q4_0)
    S = len(lens)
    rng = np.random.default_rng(0x7350 + sum(lens))
    prompts = [(rng.standard_normal((L, N)) * 0.5).astype(np.float32) for L in lens]
    rows = [(sl, p) for sl, L in enumerate(lens) for p in range(L)]
    order = rng.permutation(len(rows))
    slots = np.array([rows[i][0] for i in order], np.int32)
    pos = np.array([rows[i][1] for i in order], np.int32)
    inp = np.stack([prompts[rows[i][0]][rows[i][1]] for i in order])
    kd = torch.zeros((S, N_LAYER, H, N_POS, 64), dtype=torch.float32, device="cuda")
    vd = torch.zeros_like(kd)
    hid = torch.zeros((len(rows), N), dtype=torch.float32, device="cuda")
    say(f"t3 prefill lens={lens}")
    s.t3_prefill(dm, torch.from_numpy(slots).cuda(), torch.from_numpy(pos).cuda(), kd, vd, hid,
                 inputs=torch.from_numpy(inp).cuda())
    torch.cuda.synchronize()
    got = hid.cpu().numpy()
    kr, vr = T3.new_cache(S, N_LAYER, H, N_POS)
    pos_r = np.zeros(S, np.int64)
    want = {}
    for t in range(max(lens)):
        act = np.array([t < L for L in lens])
        x = np.stack([prompts[sl][min(t, L - 1)] for sl, L in enumerate(lens)])
        out = T3.step(rm, None, pos_r, kr, vr, inputs=x, active=act)
        for sl in np.nonzero(act)[0]:
            want[(sl, t)] = out[sl]
    ref = np.stack([want[(int(a), int(b))] for a, b in zip(slots, pos)])
    ok, err = close(got, ref)
    assert ok, f"prefill: max err {err:.3g}"
    # decode from the prefilled caches
    pos_d = torch.from_numpy(np.array(lens, np.int32)).cuda()
    hd = torch.zeros((S, N), dtype=torch.float32, device="cuda")
    for t in range(2):
        toks = rng.integers(0, V, S).astype(np.int32)
        s.t3_step(dm, pos_d, kd, vd, hd, tokens=torch.from_numpy(toks).cuda())
        torch.cuda.synchronize()
        w = T3.step(rm, toks, pos_r, kr, vr)
        ok, err = close(hd.cpu().numpy(), w)
        assert ok, f"decode {t}: max err {err:.3g}"


def planted_caches(torch, B, n_layer, n_ctx, seed):
    """Device caches [B][n_layer][H][n_ctx][64] of seeded N(0, 0.5) values, as
    if earlier positions had been decoded; every 97th position's k rows are
    8x larger, so scores far above or below the rest turn up late in a
    run and the running softmax has to rescale what it has summed."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    kd = torch.randn((B, n_layer, H, n_ctx, 64), generator=g, device="cuda") * 0.5
    vd = torch.randn((B, n_layer, H, n_ctx, 64), generator=g, device="cuda") * 0.5
    kd[:, :, :, 13::97] *= 8.0
    return kd, vd


def host_caches(kd, vd, lengths):
    """The oracle's copy of each stream's first lengths[r] positions (fp32,
    as the device holds them)."""
    kr = T3.StreamCaches([kd[r, :, :, :L].cpu().numpy() for r, L in enumerate(lengths)])
    vr = T3.StreamCaches([vd[r, :, :, :L].cpu().numpy() for r, L in enumerate(lengths)])
    return kr, vr


# Positions past which each attention variant runs more than one batch per
# wave (so the running softmax rescales across batches and the batch loop's
# clamped tail loads are used): t3_attn<6,4> (16 streams and more: 4 waves, 24
# positions per wave per batch) past 96, t3_attn<6,16> (rows x heads under
# 256: 16 waves) past 384; n_ctx - 1 is the last slot of the cache.
LONG_POSITIONS = {
    16: [0, 1, 95, 96, 97, 98, 191, 200, 385, 500, 777, 1000, 1500, 2047, 3001, N_CTX_LONG - 1],
    5: [384, 385, 1000, 2500, 4000],
    1: [N_CTX_LONG - 2],
}


@pytest.mark.parametrize("B", sorted(LONG_POSITIONS))
def test_t3_step_long_context(cbx, torch_cuda, B):
    """One cbx_t3_step per stream at positions up to n_ctx - 1 in caches of
    4096 positions (24 layers, Q4_0), the positions before each stream's
    planted, several positions per call; then a second step, where a stream
    at n_ctx - 1 has run out of cache and sits out (zero row, position
    unchanged).  16 streams run the 4-wave attention and the matrix cores,
    5 the 16-wave attention and the mat-vec, 1 the 16-wave attention and the
    mat-vec with folded norms."""
    torch = torch_cuda
    mod, s = cbx
    dm, rm = model(torch, mod, O.WTYPE_Q4_0, n_pos=N_CTX_LONG)
    P = np.array(LONG_POSITIONS[B], np.int64)
    say(f"t3 long context B={B} positions {P.min()}..{P.max()}")
    kd, vd = planted_caches(torch, B, N_LAYER, N_CTX_LONG, 0x7360 + B)
    kr, vr = host_caches(kd, vd, np.minimum(P + 2, N_CTX_LONG))
    pos_d = torch.from_numpy(P.astype(np.int32)).cuda()
    pos_r = P.copy()
    hid = torch.zeros((B, N), dtype=torch.float32, device="cuda")
    rng = np.random.default_rng(0x7361 + B)
    worst = 0.0
    for t in range(2):
        toks = rng.integers(0, V, B).astype(np.int32)
        act = pos_r < N_CTX_LONG
        say(f"  step {t}")
        s.t3_step(dm, pos_d, kd, vd, hid, tokens=torch.from_numpy(toks).cuda())
        torch.cuda.synchronize()
        want = T3.step(rm, toks, pos_r, kr, vr, active=act)
        got = hid.cpu().numpy()
        ok, err = close(got, want)
        worst = max(worst, err)
        assert ok, f"step {t}: max err {err:.3g}"
        assert np.all(got[~act] == 0.0)
        assert np.array_equal(pos_d.cpu().numpy(), pos_r)
    if B == 16:
        assert (pos_r == N_CTX_LONG).sum() == 1
    say(f"  max |err| {worst:.3g}")
    del kd, vd
    torch.cuda.empty_cache()


def test_t3_prefill_long_then_decode(cbx, torch_cuda):
    """The prompt pass at lengths where the 2-wave prompt attention runs
    several batches per wave: stream 0's 320-position prompt from position
    0, and stream 1's 130 rows continuing a planted 150-position cache (a
    prompt fed in two calls), 450 rows shuffled in one cbx_t3_prefill call
    (matrix cores), against the oracle's one-pass prompt; then two decode
    steps of both streams (mat-vec with folded norms, 16-wave attention)."""
    torch = torch_cuda
    mod, s = cbx
    n_ctx = 1024
    dm, rm = model(torch, mod, O.WTYPE_Q4_0, n_pos=N_CTX_LONG)
    rng = np.random.default_rng(0x7370)
    kd, vd = planted_caches(torch, 2, N_LAYER, n_ctx, 0x7371)
    kd[0].zero_()
    vd[0].zero_()
    starts, lens = (0, 150), (320, 130)
    kr, vr = T3.new_cache(2, N_LAYER, H, 330)
    kr[1, :, :, :150] = kd[1, :, :, :150].cpu().numpy()
    vr[1, :, :, :150] = vd[1, :, :, :150].cpu().numpy()
    prompts = [(rng.standard_normal((L, N)) * 0.5).astype(np.float32) for L in lens]
    rows = [(sl, starts[sl] + i) for sl in range(2) for i in range(lens[sl])]
    order = rng.permutation(len(rows))
    slots = np.array([rows[i][0] for i in order], np.int32)
    pos = np.array([rows[i][1] for i in order], np.int32)
    inp = np.stack([prompts[rows[i][0]][rows[i][1] - starts[rows[i][0]]] for i in order])
    hid = torch.zeros((len(rows), N), dtype=torch.float32, device="cuda")
    say(f"t3 long prefill rows={len(rows)}")
    s.t3_prefill(dm, torch.from_numpy(slots).cuda(), torch.from_numpy(pos).cuda(), kd, vd, hid,
                 inputs=torch.from_numpy(inp).cuda())
    torch.cuda.synchronize()
    want = {}
    for sl in range(2):
        out = T3.prefill(rm, prompts[sl], kr, vr, sl, starts[sl])
        for i in range(lens[sl]):
            want[(sl, starts[sl] + i)] = out[i]
    ref = np.stack([want[(int(a), int(b))] for a, b in zip(slots, pos)])
    ok, err = close(hid.cpu().numpy(), ref)
    assert ok, f"prefill: max err {err:.3g}"
    say(f"  prefill max |err| {err:.3g}")
    pos_d = torch.tensor([320, 280], dtype=torch.int32, device="cuda")
    pos_r = np.array([320, 280], np.int64)
    hd = torch.zeros((2, N), dtype=torch.float32, device="cuda")
    for t in range(2):
        toks = rng.integers(0, V, 2).astype(np.int32)
        s.t3_step(dm, pos_d, kd, vd, hd, tokens=torch.from_numpy(toks).cuda())
        torch.cuda.synchronize()
        w = T3.step(rm, toks, pos_r, kr, vr)
        ok, err = close(hd.cpu().numpy(), w)
        assert ok, f"decode {t}: max err {err:.3g}"
    del kd, vd
    torch.cuda.empty_cache()
