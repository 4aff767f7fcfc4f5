"""The T3 transformer reader (cbx_gguf_read_t3 / cbx_gguf_load_t3,
chatterbox.cpp_amd/csrc/cbx_gguf.cpp) on files from the separate test writer
(tests/gguf_writer.py), with the tensor names and types
scripts/convert-t3-turbo-to-gguf.py:150-189 writes (speech_emb F16, matrices
F16 / Q4_0 / Q8_0, the rest F32) and the keys main.cpp:356-367 requires.
CPU only: the parse; the load runs on the GPU (tests/test_gpu_t3.py).
"""
import numpy as np
import pytest

import gguf_writer as G
import oracle_lib as O
import pkg

GGML = {O.WTYPE_F16: G.GGML_F16, O.WTYPE_Q4_0: G.GGML_Q4_0, O.WTYPE_Q5_0: G.GGML_Q5_0,
        O.WTYPE_Q8_0: G.GGML_Q8_0}


@pytest.fixture(scope="module")
def mod():
    return pkg.load()


def make_t3(rng, *, n_layer=2, n=256, H=4, n_pos=32, V=300, wtype=O.WTYPE_Q8_0, emb_f16=True,
            eps=1e-5, drop=(), override=None, kv_override=None):
    """A T3 GGUF: returns (file bytes, the tensors' values as the format
    defines them, keyed like oracle/cbx_t3_oracle.py's Model).  drop: tensor
    or key names left out; override: {name: (ne, ggml type, raw)}."""
    override = override or {}
    kvs = {"chatterbox.n_ctx": (G.U32, n_pos), "chatterbox.n_embd": (G.U32, n),
           "chatterbox.n_head": (G.U32, H), "chatterbox.n_layer": (G.U32, n_layer),
           "chatterbox.speech_vocab_size": (G.U32, V),
           "chatterbox.start_speech_token": (G.U32, V - 2),
           "chatterbox.stop_speech_token": (G.U32, V - 1),
           "chatterbox.layer_norm_eps": (G.F32, eps)}
    kvs.update(kv_override or {})
    tensors, vals = [], {"layers": []}

    def vec(name, k, base=0.0, sd=0.1):
        a = (base + rng.standard_normal(k) * sd).astype(np.float32)
        tensors.append((name, (k,), G.GGML_F32, a.tobytes()))
        return a

    def mat(name, o, i):
        w = (rng.standard_normal((o, i)) * 0.05).astype(np.float32)
        blocks = O.quantize(w, wtype)
        tensors.append((name, (i, o), GGML[wtype], blocks.tobytes()))
        return O.dequantize(blocks, wtype, i)

    wpe = (rng.standard_normal((n_pos, n)) * 0.1).astype(np.float32)
    tensors.append(("model/wpe", (n, n_pos), G.GGML_F32, wpe.tobytes()))
    emb = (rng.standard_normal((V, n)) * 0.5).astype(np.float16 if emb_f16 else np.float32)
    tensors.append(("chatterbox/speech_emb", (n, V), G.GGML_F16 if emb_f16 else G.GGML_F32,
                    emb.tobytes()))
    vals["wpe"], vals["speech_emb"] = wpe, emb.astype(np.float32)
    vals["ln_f_g"], vals["ln_f_b"] = vec("model/ln_f/g", n, 1.0), vec("model/ln_f/b", n)
    for l in range(n_layer):
        p = f"model/h{l}/"
        L = {}
        L["ln_1_g"], L["ln_1_b"] = vec(p + "ln_1/g", n, 1.0), vec(p + "ln_1/b", n)
        L["attn_w"], L["attn_b"] = mat(p + "attn/c_attn/w", 3 * n, n), vec(p + "attn/c_attn/b", 3 * n, 0, 0.02)
        L["attn_proj_w"] = mat(p + "attn/c_proj/w", n, n)
        L["attn_proj_b"] = vec(p + "attn/c_proj/b", n, 0, 0.02)
        L["ln_2_g"], L["ln_2_b"] = vec(p + "ln_2/g", n, 1.0), vec(p + "ln_2/b", n)
        L["fc_w"], L["fc_b"] = mat(p + "mlp/c_fc/w", 4 * n, n), vec(p + "mlp/c_fc/b", 4 * n, 0, 0.02)
        L["fc_proj_w"] = mat(p + "mlp/c_proj/w", n, 4 * n)
        L["fc_proj_b"] = vec(p + "mlp/c_proj/b", n, 0, 0.02)
        vals["layers"].append(L)
    tensors = [(nm,) + override[nm] if nm in override else (nm, ne, ty, raw)
               for nm, ne, ty, raw in tensors if nm not in drop]
    kv_list = [("general.architecture", G.STRING, "chatterbox")] + [
        (k, t, v) for k, (t, v) in kvs.items() if k not in drop]
    data, data0, _ = G.build(kv_list, tensors)
    vals["data0"] = data0
    return data, vals


def _write(tmp_path, data, name="t3.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def _code(mod, path):
    try:
        mod.read_t3_gguf(path)
    except mod.CbxError as e:
        return e.code
    return 0


@pytest.mark.parametrize("wtype", [O.WTYPE_F16, O.WTYPE_Q4_0, O.WTYPE_Q5_0, O.WTYPE_Q8_0])
def test_reads_the_t3_model(mod, tmp_path, wtype):
    rng = np.random.default_rng(31 + wtype)
    data, _ = make_t3(rng, wtype=wtype, emb_f16=wtype != O.WTYPE_F16)
    info = mod.read_t3_gguf(_write(tmp_path, data))
    n, L = 256, 2
    assert (info.n_layer, info.n_embd, info.n_head, info.n_pos, info.n_speech_vocab) == (L, n, 4, 32, 300)
    assert info.wtype == wtype and info.eps == np.float32(1e-5)
    assert (info.start_speech_token, info.stop_speech_token, info.gguf_version) == (298, 299, 3)
    bb = {O.WTYPE_F16: 64, O.WTYPE_Q4_0: 18, O.WTYPE_Q5_0: 22, O.WTYPE_Q8_0: 34}[wtype]
    r = lambda x: (x + 255) // 256 * 256
    want = r(4 * n * 32) + r(4 * n * 300) + 2 * r(4 * n)
    want += L * (4 * r(4 * n) + r(4 * 3 * n) + 2 * r(4 * n) + r(4 * 4 * n)
                 + r(3 * n * n // 32 * bb) + r(n * n // 32 * bb) + r(4 * n * n // 32 * bb)
                 + r(n * 4 * n // 32 * bb))
    assert info.device_bytes == want


def test_rejects_damaged_and_mismatched_files(mod, tmp_path):
    rng = np.random.default_rng(37)
    INV, UNS = mod.CBX_ERR_INVALID, mod.CBX_ERR_UNSUPPORTED
    cases = [
        (dict(drop=("chatterbox.n_layer",)), INV),
        (dict(drop=("chatterbox.layer_norm_eps",)), INV),
        (dict(drop=("model/h1/mlp/c_fc/b",)), INV),
        (dict(kv_override={"chatterbox.n_ctx": (G.U32, 33)}), INV),          # wpe rows differ
        (dict(kv_override={"chatterbox.speech_vocab_size": (G.U32, 299)}), INV),
        (dict(kv_override={"chatterbox.layer_norm_eps": (G.F32, -1.0)}), INV),
        (dict(kv_override={"chatterbox.n_head": (G.U32, 2)}), UNS),          # 128-wide heads
        (dict(kv_override={"chatterbox.n_layer": (G.U32, 3)}), INV),         # no layer 2
        (dict(override={"model/h0/attn/c_attn/w": ((256, 700), G.GGML_Q8_0,
                                                    bytes(700 * 8 * 34))}), INV),
        (dict(override={"model/h1/attn/c_proj/w": ((256, 256), G.GGML_Q4_0,
                                                    bytes(256 * 8 * 18))}), UNS),  # mixed types
        (dict(override={"model/h0/ln_1/g": ((256,), G.GGML_F16, bytes(512))}), INV),
    ]
    for kw, code in cases:
        data, _ = make_t3(rng, **kw)
        assert _code(mod, _write(tmp_path, data)) == code, kw
    # every matrix in a format the kernels do not take (Q4_1: 20-byte blocks)
    q41 = {}
    for l in range(2):
        for nm, (i, o) in (("attn/c_attn/w", (256, 768)), ("attn/c_proj/w", (256, 256)),
                           ("mlp/c_fc/w", (256, 1024)), ("mlp/c_proj/w", (1024, 256))):
            q41[f"model/h{l}/{nm}"] = ((i, o), 3, bytes(o * i // 32 * 20))
    data, _ = make_t3(rng, override=q41)
    assert _code(mod, _write(tmp_path, data)) == UNS


def test_truncations_fail_cleanly(mod, tmp_path):
    """A small file cut at about 400 places (through the header and tensor
    infos, then spread over the data): each cut is CBX_ERR_INVALID."""
    rng = np.random.default_rng(41)
    data, vals = make_t3(rng, n_layer=1, n_pos=4, V=8)
    d0 = vals["data0"]  # the end of the header and tensor infos
    cuts = sorted(set(list(range(0, d0, max(1, d0 // 340))) +
                      list(np.linspace(d0, len(data) - 1, 60).astype(int))))
    assert len(cuts) >= 390
    for c in cuts:
        p = _write(tmp_path, data[:c], "cut.gguf")
        assert _code(mod, p) == mod.CBX_ERR_INVALID, c
    assert _code(mod, _write(tmp_path, data, "whole.gguf")) == 0
