"""GPU parity of the fused speech_head variant (cbx_head_logits /
cbx_head_sample_batch, chatterbox.cpp_amd/csrc/cbx_head.hip) against the
oracle: the projection against the oracle's binary64 head (W dequantized
exactly as the format defines, main.cpp:577) within a bound on binary32
accumulation, and the fused call's tokens against the oracle sampler run on
the logits the GPU projected (bit-exact, as for any logits).

Tolerance: |gpu - ref| <= 1e-5 * sum_k |w_vk h_rk|
+ 2^-39 * max_k |h_rk| * sum_k |w_vk| + 1e-6 per logit (fp32 products and sums
over n_embd terms; the middle term is the matrix-core path's split floor,
2^-39 of the row's largest magnitude per activation, about 1e-10 for rows of
ordinary range; a term lost or misplaced moves a logit by about sum |w h| /
n_embd, a hundred times the bound).
"""
import numpy as np
import pytest

import oracle_lib as O
import pkg

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="module")
def cbx(torch_cuda):
    mod = pkg.load()
    s = mod.Sampler(0, 32768, 1024)
    yield mod, s
    s.close()


def _problem(rng, V, K, R, wtype, scale=0.05):
    w = (rng.standard_normal((V, K)) * scale).astype(np.float32)
    blocks = O.quantize(w, wtype)
    bias = (rng.standard_normal(V) * 0.1).astype(np.float32)
    h = rng.standard_normal((R, K)).astype(np.float32)
    return blocks, bias, h


def _tol(blocks, wtype, h, K):
    deq = np.abs(O.dequantize(blocks, wtype, K)).astype(np.float64)
    ah = np.abs(h).astype(np.float64)
    floor = 2.0 ** -39 * ah.max(axis=1)[:, None] * deq.sum(axis=1)[None, :]
    return 1e-5 * (ah @ deq.T) + floor + 1e-6


def _gpu_head(cbx, torch, blocks, wtype, bias, h, V, K, ld, ld_h=None):
    mod, s = cbx
    R = h.shape[0]
    ld_h = K if ld_h is None else ld_h
    hp = np.zeros((R, ld_h), np.float32)
    hp[:, :K] = h
    dW = torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)).cuda()
    dh = torch.from_numpy(hp).cuda()
    db = None if bias is None else torch.from_numpy(bias).cuda()
    out = torch.full((R, ld), -7.0, dtype=torch.float32, device="cuda")
    head = mod.Sampler.head(dW, wtype, K, dh, out, bias=db)
    s.head_logits(head, R, V, ld)
    torch.cuda.synchronize()
    return out.cpu().numpy()


CASES = [
    # wtype, V, K, R, ld
    (O.WTYPE_Q4_0, 6563, 1024, 128, 6563),   # B=64 CFG pairs of the Turbo vocab
    (O.WTYPE_Q8_0, 6563, 1024, 128, 6576),
    (O.WTYPE_F16, 6563, 1024, 40, 6563),
    (O.WTYPE_Q4_0, 8194, 1024, 2, 8194),     # one CFG pair, the Llama vocab
    (O.WTYPE_Q8_0, 300, 64, 17, 301),        # ragged tiles on both axes
    (O.WTYPE_F16, 33, 32, 1, 40),
    # fewer than 16 rows: the mat-vec kernel
    (O.WTYPE_Q4_0, 6563, 1024, 1, 6563),     # one stream of the Turbo vocab
    (O.WTYPE_Q8_0, 6563, 1024, 2, 6570),
    (O.WTYPE_F16, 6563, 1024, 2, 6563),
    (O.WTYPE_Q4_0, 6563, 1024, 15, 6563),    # the largest mat-vec batch
    (O.WTYPE_Q8_0, 1000, 4096, 3, 1000),
    (O.WTYPE_Q4_0, 300, 64, 5, 301),
    (O.WTYPE_F16, 500, 8192, 1, 500),
    (O.WTYPE_Q4_0, 700, 512, 16, 700),       # 16 rows: the matrix-core tiles again
    (O.WTYPE_Q5_0, 6563, 1024, 128, 6563),   # Q5_0 (--quant q5_0): the matrix cores
    (O.WTYPE_Q5_0, 300, 64, 17, 301),        #   ragged tiles on both axes
    (O.WTYPE_Q5_0, 6563, 1024, 2, 6563),     #   the mat-vec, one CFG pair
    (O.WTYPE_Q5_0, 1000, 4096, 3, 1000),     #   the mat-vec, long rows
]


@pytest.mark.parametrize("case", CASES, ids=[f"w{c[0]}_V{c[1]}_K{c[2]}_R{c[3]}" for c in CASES])
def test_head_logits_against_f64(cbx, torch_cuda, case):
    wtype, V, K, R, ld = case
    rng = np.random.default_rng(V * 7 + R + wtype)
    blocks, bias, h = _problem(rng, V, K, R, wtype)
    say(f"head wtype={wtype} V={V} K={K} R={R}")
    got = _gpu_head(cbx, torch_cuda, blocks, wtype, bias, h, V, K, ld, ld_h=K + 3 * (R % 2))
    ref = O.head_f64(blocks, wtype, bias, h, V, K)
    tol = _tol(blocks, wtype, h, K)
    err = np.abs(got[:, :V].astype(np.float64) - ref)
    assert np.all(err <= tol), f"max err {err.max():.3g}, worst ratio {(err / tol).max():.3g}"
    if ld > V:
        assert np.all(got[:, V:] == -7.0), "stores past n_vocab"


@pytest.mark.parametrize("wtype", [O.WTYPE_Q4_0, O.WTYPE_Q5_0, O.WTYPE_Q8_0, O.WTYPE_F16])
def test_head_from_gguf(cbx, torch_cuda, tmp_path, wtype):
    """cbx_gguf_read_head + cbx_gguf_load_head (csrc/cbx_gguf.cpp) put the
    file's speech_head and bias in device memory byte for byte, and the
    projection of the loaded head matches the oracle's."""
    import gguf_writer as G
    mod, s = cbx
    torch = torch_cuda
    V, K, R = 700, 256, 24
    rng = np.random.default_rng(40 + wtype)
    blocks, bias, h = _problem(rng, V, K, R, wtype)
    gt = {O.WTYPE_Q4_0: G.GGML_Q4_0, O.WTYPE_Q5_0: G.GGML_Q5_0, O.WTYPE_Q8_0: G.GGML_Q8_0,
          O.WTYPE_F16: G.GGML_F16}[wtype]
    data, _, _ = G.t3_head_file(blocks, gt, K, bias, stop=V - 1, start=V - 2)
    path = tmp_path / "head.gguf"
    path.write_bytes(data)
    say(f"gguf head wtype={wtype} V={V} K={K}")
    info, dW, db = mod.load_head_gguf(str(path))
    assert (info.n_vocab, info.n_embd, info.wtype, info.stop_speech_token) == (V, K, wtype, V - 1)
    assert dW.cpu().numpy().tobytes() == np.ascontiguousarray(blocks).tobytes()
    assert np.array_equal(db.cpu().numpy(), bias)
    dh = torch.from_numpy(h).cuda()
    out = torch.full((R, V), -7.0, dtype=torch.float32, device="cuda")
    head = mod.Sampler.head(dW, info.wtype, info.n_embd, dh, out, bias=db)
    s.head_logits(head, R, info.n_vocab, V)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = O.head_f64(blocks, wtype, bias, h, V, K)
    tol = _tol(blocks, wtype, h, K)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= tol)


@pytest.mark.parametrize("wtype", [O.WTYPE_Q4_0, O.WTYPE_Q5_0, O.WTYPE_Q8_0, O.WTYPE_F16])
def test_head_row_magnitudes(cbx, torch_cuda, wtype):
    """The matrix-core path scales each activation row by its own power of two
    before splitting it into two fp16 parts: rows of magnitude 1e6 (past the
    fp16 range), 1e-6 (below its normal range), 1e35, all zeros, mixed rows
    (one 1e5 entry among ordinary ones) and rows holding the largest finite
    float all project as the binary64 head does, within the same bound."""
    V, K, R = 900, 512, 32
    rng = np.random.default_rng(77 + wtype)
    blocks, bias, h = _problem(rng, V, K, R, wtype)
    h[0:8] *= 1e6
    h[8:16] *= 1e-6
    h[16:20] = 0.0
    h[20:24, 7] = 1e5
    h[24:28] *= 1e35
    h[28, 3] = np.finfo(np.float32).max
    h[29, 4] = -np.finfo(np.float32).max
    say(f"head row magnitudes wtype={wtype} V={V} K={K} R={R}")
    got = _gpu_head(cbx, torch_cuda, blocks, wtype, bias, h, V, K, V)
    ref = O.head_f64(blocks, wtype, bias, h, V, K)
    tol = _tol(blocks, wtype, h, K)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= tol), f"max err {err.max():.3g}, worst ratio {(err / tol).max():.3g}"
    assert np.array_equal(got[16:20], np.broadcast_to(bias, (4, V)))  # zero rows: the bias


def test_head_without_bias(cbx, torch_cuda):
    rng = np.random.default_rng(5)
    blocks, _, h = _problem(rng, 500, 256, 20, O.WTYPE_Q4_0)
    got = _gpu_head(cbx, torch_cuda, blocks, O.WTYPE_Q4_0, None, h, 500, 256, 500)
    ref = O.head_f64(blocks, O.WTYPE_Q4_0, None, h, 500, 256)
    tol = _tol(blocks, O.WTYPE_Q4_0, h, 256)
    assert np.all(np.abs(got - ref) <= tol)


@pytest.mark.parametrize("B,S", [(64, 2), (1, 1), (7, 1)])
@pytest.mark.parametrize("wtype", [O.WTYPE_Q4_0, O.WTYPE_Q5_0, O.WTYPE_Q8_0, O.WTYPE_F16])
def test_fused_head_sample_cfg(cbx, torch_cuda, wtype, B, S):
    """B CFG streams, S steps: projection of cond and uncond hidden rows
    (weights from N(0, 0.02), hidden rows N(0, 1)), then the sampler (k 1000,
    p 0.95, T 0.8, pen 1.2, w 0.5) in one call.  B=64 x 2 projects 256 rows
    on the matrix cores; one CFG pair (2 rows) and 7 pairs (14 rows) take the
    mat-vec kernel."""
    torch = torch_cuda
    mod, s = cbx
    V, K = 6563, 1024
    rng = np.random.default_rng(77 + wtype)
    blocks, bias, h = _problem(rng, V, K, B * S, wtype, scale=0.02)
    hu = (h + 0.5 * rng.standard_normal(h.shape)).astype(np.float32)
    hist = rng.integers(0, V, size=(B, 300)).astype(np.int32)
    hl = rng.integers(0, 301, size=B).astype(np.int32)
    plist = [dict(top_k=1000, top_p=0.95, temp=0.8, repeat_penalty=1.2, min_p=0.0,
                  cfg_weight=0.5)] * B
    u = rng.random(B * S)
    w = pkg.workloads()
    dW = torch.from_numpy(blocks.reshape(-1)).cuda()
    dh, dhu = torch.from_numpy(h).cuda(), torch.from_numpy(hu).cuda()
    lc = torch.zeros((B * S, V), dtype=torch.float32, device="cuda")
    lu = torch.zeros_like(lc)
    head = mod.Sampler.head(dW, wtype, K, dh, lc, bias=torch.from_numpy(bias).cuda(),
                            hidden_uncond=dhu, logits_uncond=lu)
    prm = torch.from_numpy(w.pack_params(plist)).cuda()
    tok = torch.full((B * S,), -5, dtype=torch.int32, device="cuda")
    info = torch.zeros(B * S, dtype=torch.int32, device="cuda")
    say(f"fused head+sample wtype={wtype} B={B} S={S}")
    s.head_sample_batch(head, lc, prm, tok, n_steps=S, info=info,
                        uniforms=torch.from_numpy(u).cuda(),
                        history=torch.from_numpy(hist).cuda(),
                        history_len=torch.from_numpy(hl).cuda(), max_survivors=1024)
    torch.cuda.synchronize()
    got = tok.cpu().numpy()
    lcn, lun = lc.cpu().numpy(), lu.cpu().numpy()
    # the projection is the head's
    for x, hh in ((lcn, h), (lun, hu)):
        ref = O.head_f64(blocks, wtype, bias, hh, V, K)
        assert np.all(np.abs(x - ref) <= _tol(blocks, wtype, hh, K))
    # and the tokens are the oracle sampler's on those logits
    op = [O.params(**p) for p in plist] * S
    want = np.array([O.sample_row(lcn[r], hist[r % B][: hl[r % B]], op[r], u[r],
                                  uncond=lun[r])[0] for r in range(B * S)])
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:8]


def test_head_rejects_bad_arguments(cbx, torch_cuda):
    torch = torch_cuda
    mod, s = cbx
    dW = torch.zeros(18 * 32, dtype=torch.uint8, device="cuda")
    dh = torch.zeros((2, 64), dtype=torch.float32, device="cuda")
    out = torch.zeros((2, 16), dtype=torch.float32, device="cuda")
    for wtype, K in ((3, 64), (O.WTYPE_Q4_0, 48), (O.WTYPE_Q4_0, 0)):
        head = mod.Sampler.head(dW, wtype, K, dh, out)
        with pytest.raises(mod.CbxError):
            s.head_logits(head, 2, 16, 16)
    head = mod.Sampler.head(dW, O.WTYPE_Q4_0, 64, dh, out)
    with pytest.raises(mod.CbxError):
        s.head_logits(head, 2, 16, 8)  # ld_logits < n_vocab
