"""cbx_gguf_read_head (chatterbox.cpp_amd/csrc/cbx_gguf.cpp, include/cbx_gguf.h)
on GGUF files written by tests/gguf_writer.py: the speech_head, its bias and
the chatterbox.* keys the reference loader reads (src/main.cpp:356-399,
src/chatterbox_t3_internal.h:33-40), as scripts/convert-t3-turbo-to-gguf.py
writes them.  CPU only: the parse makes no HIP call, and the load is checked
here only for its argument errors (tests/test_gpu_head.py loads to a GPU).

The reader is pinned by the published layout (the writer is separate code),
by the byte offsets it reports (the bytes there are the bytes written), and
by damaged files: every truncation of a small file and seeded byte flips must
end in an error code or a consistent result, never a crash or a read past
the file.
"""
import os

import numpy as np
import pytest

import gguf_writer as G
import oracle_lib as O
import pkg

CBX_ERR_INVALID, CBX_ERR_UNSUPPORTED = -1, -3


@pytest.fixture(scope="module")
def mod():
    return pkg.load()


def _blocks(rng, wtype, V, K):
    w = (rng.standard_normal((V, K)) * 0.05).astype(np.float32)
    return O.quantize(w, wtype)


def _write(tmp_path, data, name="t3.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def _code(mod, path):
    try:
        mod.read_head_gguf(path)
    except mod.CbxError as e:
        return e.code
    return 0


@pytest.mark.parametrize("wtype,ggml_type,V,K", [
    (O.WTYPE_Q4_0, G.GGML_Q4_0, 6563, 1024),   # the Turbo head, --quant q4_0
    (O.WTYPE_Q8_0, G.GGML_Q8_0, 300, 64),
    (O.WTYPE_Q5_0, G.GGML_Q5_0, 6563, 1024),   # --quant q5_0
    (O.WTYPE_F16, G.GGML_F16, 8194, 64),       # F16, the converter's default
])
def test_reads_the_head(mod, tmp_path, wtype, ggml_type, V, K):
    rng = np.random.default_rng(V + K)
    blocks = _blocks(rng, wtype, V, K)
    bias = rng.standard_normal(V).astype(np.float32)
    data, data0, offs = G.t3_head_file(blocks, ggml_type, K, bias, stop=V - 1, start=V - 2)
    path = _write(tmp_path, data)
    info = mod.read_head_gguf(path)
    assert (info.n_vocab, info.n_embd, info.wtype, info.has_bias) == (V, K, wtype, 1)
    assert (info.speech_vocab_size, info.stop_speech_token, info.start_speech_token) == (V, V - 1, V - 2)
    assert info.gguf_version == 3
    raw = np.ascontiguousarray(blocks).tobytes()
    assert info.weight_bytes == len(raw)
    assert info.weight_offset == data0 + offs[1]
    assert data[info.weight_offset:info.weight_offset + info.weight_bytes] == raw
    assert info.bias_bytes == 4 * V
    assert data[info.bias_offset:info.bias_offset + info.bias_bytes] == bias.tobytes()


def test_version_2_alignment_and_absent_keys(mod, tmp_path):
    rng = np.random.default_rng(5)
    blocks = _blocks(rng, O.WTYPE_Q4_0, 40, 32)
    kvs = [("general.name", G.STRING, "x")]
    tensors = [("chatterbox/speech_head", (32, 40), G.GGML_Q4_0, blocks.tobytes())]
    data, data0, offs = G.build(kvs, tensors, version=2, alignment=256)
    assert data0 % 256 == 0
    info = mod.read_head_gguf(_write(tmp_path, data))
    assert (info.gguf_version, info.n_vocab, info.has_bias) == (2, 40, 0)
    assert (info.speech_vocab_size, info.stop_speech_token, info.start_speech_token) == (-1, -1, -1)
    assert (info.bias_offset, info.bias_bytes) == (0, 0)
    assert data[info.weight_offset:info.weight_offset + info.weight_bytes] == blocks.tobytes()


def test_bias_as_a_column(mod, tmp_path):
    rng = np.random.default_rng(6)
    blocks = _blocks(rng, O.WTYPE_Q8_0, 10, 32)
    bias = np.arange(10, dtype=np.float32)
    tensors = [("chatterbox/speech_head", (32, 10), G.GGML_Q8_0, blocks.tobytes()),
               ("chatterbox/speech_head_bias", (10, 1), G.GGML_F32, bias.tobytes())]
    data, _, _ = G.build([], tensors)
    info = mod.read_head_gguf(_write(tmp_path, data))
    assert info.has_bias == 1 and data[info.bias_offset:info.bias_offset + 40] == bias.tobytes()


def _small(rng, **kw):
    blocks = _blocks(rng, O.WTYPE_Q4_0, 8, 64)
    bias = rng.standard_normal(8).astype(np.float32)
    return G.t3_head_file(blocks, G.GGML_Q4_0, 64, bias, stop=7, start=6, **kw)


def test_rejects_damaged_and_mismatched_files(mod, tmp_path):
    rng = np.random.default_rng(7)
    good, _, _ = _small(rng)
    assert _code(mod, _write(tmp_path, good)) == 0
    blocks = _blocks(rng, O.WTYPE_Q4_0, 8, 64)
    bias = np.zeros(8, np.float32)
    cases = {
        "magic": (G.build([], [], magic=b"GGUG")[0], CBX_ERR_INVALID),
        "version 1": (G.build([], [], version=1)[0], CBX_ERR_UNSUPPORTED),
        "version 4": (G.build([], [], version=4)[0], CBX_ERR_UNSUPPORTED),
        "no head": (G.build([("a", G.U32, 1)], [])[0], CBX_ERR_INVALID),
        "Q4_1 head": (G.build([], [("chatterbox/speech_head", (64, 8), 3,
                                    b"\0" * 20 * 2 * 8)])[0], CBX_ERR_UNSUPPORTED),
        "F32 head": (G.build([], [("chatterbox/speech_head", (64, 8), G.GGML_F32,
                                   b"\0" * 4 * 64 * 8)])[0], CBX_ERR_UNSUPPORTED),
        "3-D head": (G.build([], [("chatterbox/speech_head", (64, 8, 1), G.GGML_Q4_0,
                                   blocks.tobytes())])[0], CBX_ERR_INVALID),
        "n_embd 48": (G.build([], [("chatterbox/speech_head", (48, 8), G.GGML_F16,
                                    b"\0" * 2 * 48 * 8)])[0], CBX_ERR_INVALID),
        "vocab too large": (G.build([], [("chatterbox/speech_head", (32, 40000), G.GGML_Q4_0,
                                          b"")], offsets=[0])[0], CBX_ERR_INVALID),
        "speech_vocab_size differs": (G.t3_head_file(blocks, G.GGML_Q4_0, 64, bias, vocab=9,
                                                     stop=3)[0], CBX_ERR_INVALID),
        "stop token past the vocab": (G.t3_head_file(blocks, G.GGML_Q4_0, 64, bias,
                                                     stop=8)[0], CBX_ERR_INVALID),
        "n_embd key differs": (G.build([("chatterbox.n_embd", G.U32, 32)],
                                       [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                         blocks.tobytes())])[0], CBX_ERR_INVALID),
        "key of the wrong type": (G.build([("chatterbox.stop_speech_token", G.STRING, "6562")],
                                          [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                            blocks.tobytes())])[0], CBX_ERR_INVALID),
        "negative stop token": (G.build([("chatterbox.stop_speech_token", G.I32, -2)],
                                        [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                          blocks.tobytes())])[0], CBX_ERR_INVALID),
        "alignment 24": (G.build([], [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                       blocks.tobytes())], alignment=24)[0], CBX_ERR_INVALID),
        "bias length": (G.build([], [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                      blocks.tobytes()),
                                     ("chatterbox/speech_head_bias", (7,), G.GGML_F32,
                                      b"\0" * 28)])[0], CBX_ERR_INVALID),
        "bias of 2 x 2^63+1": (G.build([], [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                             blocks.tobytes()),
                                            ("chatterbox/speech_head_bias",
                                             (8, (1 << 63) + 1, (1 << 63) + 1), G.GGML_F32,
                                             b"\0" * 32)])[0], CBX_ERR_INVALID),
        "bias F16": (G.build([], [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                   blocks.tobytes()),
                                  ("chatterbox/speech_head_bias", (8,), G.GGML_F16,
                                   b"\0" * 16)])[0], CBX_ERR_INVALID),
        "two heads": (G.build([], [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                    blocks.tobytes())] * 2)[0], CBX_ERR_INVALID),
        "unaligned data": (G.build([], [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                         blocks.tobytes())], offsets=[4])[0], CBX_ERR_INVALID),
        "data past the end": (G.build([], [("chatterbox/speech_head", (64, 8), G.GGML_Q4_0,
                                            blocks.tobytes()[:100])])[0], CBX_ERR_INVALID),
        "tensor count": (G.build([], [], n_tensors=1 << 40)[0], CBX_ERR_INVALID),
        "pair count": (G.build([], [], n_kv=3)[0], CBX_ERR_INVALID),
        "nested array": (G.build([("x", G.ARRAY, (G.ARRAY, []))], [])[0], CBX_ERR_INVALID),
    }
    # a pair of value type 13 (none such): its type field sits after the
    # 24-byte header and the 9-byte key "k"
    bad = bytearray(G.build([("k", G.U8, 1)], [])[0])
    bad[24 + 9:24 + 13] = (13).to_bytes(4, "little")
    cases["unknown value type"] = (bytes(bad), CBX_ERR_INVALID)
    got = {name: _code(mod, _write(tmp_path, data, name.replace(" ", "_") + ".gguf"))
           for name, (data, _) in cases.items()}
    want = {name: code for name, (_, code) in cases.items()}
    assert got == want


def test_missing_file_and_null_arguments(mod, tmp_path):
    assert _code(mod, str(tmp_path / "absent.gguf")) == CBX_ERR_INVALID
    lib = mod.load_library()
    assert lib.cbx_gguf_read_head(None, None) == CBX_ERR_INVALID
    info = mod.HeadFile()
    assert lib.cbx_gguf_load_head(os.fsencode(str(tmp_path / "x")), info, None, None) == CBX_ERR_INVALID


def test_every_truncation_fails_cleanly(mod, tmp_path):
    rng = np.random.default_rng(8)
    data, _, _ = _small(rng)
    path = str(tmp_path / "cut.gguf")
    for n in range(len(data)):
        with open(path, "wb") as f:
            f.write(data[:n])
        assert _code(mod, path) == CBX_ERR_INVALID, n


def test_byte_flips_never_read_past_the_file(mod, tmp_path):
    rng = np.random.default_rng(9)
    data, _, _ = _small(rng)
    path = str(tmp_path / "flip.gguf")
    size = len(data)
    for _ in range(3000):
        d = bytearray(data)
        for _ in range(int(rng.integers(1, 4))):
            d[int(rng.integers(0, size))] = int(rng.integers(0, 256))
        with open(path, "wb") as f:
            f.write(bytes(d))
        try:
            info = mod.read_head_gguf(path)
        except mod.CbxError as e:
            assert e.code in (CBX_ERR_INVALID, CBX_ERR_UNSUPPORTED)
            continue
        # accepted: what it reports lies inside the file and is self-consistent
        assert info.weight_offset + info.weight_bytes <= size
        assert info.bias_offset + info.bias_bytes <= size
        assert info.n_embd % 32 == 0 and 1 <= info.n_vocab <= 32768
        per_row = {O.WTYPE_F16: 2 * info.n_embd, O.WTYPE_Q4_0: 18 * info.n_embd // 32,
                   O.WTYPE_Q8_0: 34 * info.n_embd // 32}[info.wtype]
        assert info.weight_bytes == per_row * info.n_vocab
