"""A GGUF file writer for tests, written from ggml's published GGUF format
(version 3, little-endian): magic "GGUF", u32 version, u64 tensor count,
u64 key/value count; each pair a string key (u64 length + bytes), a u32 value
type and the value (arrays: u32 element type, u64 count, elements); each
tensor info a string name, u32 n_dims, u64 ne[n_dims] (fastest first), u32
ggml type and u64 offset into the data section; the data section starts at
the next multiple of general.alignment (default 32) and every tensor's data
starts at a multiple of it.

It is kept separate from the reader under test (chatterbox.cpp_amd/csrc/
cbx_gguf.cpp) and lets a test break any field on purpose.  The tensor and key
names the T3 files use are those of scripts/convert-t3-turbo-to-gguf.py:160-163
and :217-224 (keys also src/chatterbox_t3_internal.h:33-40).
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q5_0, GGML_Q8_0 = 0, 1, 2, 6, 8


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_SCALAR[vtype], v)


def build(kvs, tensors, *, version=3, alignment=None, magic=b"GGUF", offsets=None,
          n_tensors=None, n_kv=None):
    """kvs: [(key, vtype, value)]; tensors: [(name, ne tuple, ggml type, raw bytes)].
    offsets: optional explicit data offsets per tensor (default: packed at the
    alignment).  Returns the file bytes."""
    align = 32 if alignment is None else alignment
    kv_list = list(kvs)
    if alignment is not None:
        kv_list = [("general.alignment", U32, alignment)] + kv_list
    head = magic + struct.pack("<I", version)
    head += struct.pack("<QQ", len(tensors) if n_tensors is None else n_tensors,
                        len(kv_list) if n_kv is None else n_kv)
    for key, vt, v in kv_list:
        head += _str(key) + struct.pack("<I", vt) + _value(vt, v)
    offs = []
    pos = 0
    for i, (_, _, _, raw) in enumerate(tensors):
        if offsets is not None:
            offs.append(offsets[i])
        else:
            offs.append(pos)
            pos += (len(raw) + align - 1) // align * align
    for (name, ne, gt, _), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne))
        head += b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", gt, off)
    data0 = (len(head) + align - 1) // align * align
    end = max([o + len(t[3]) for o, t in zip(offs, tensors)] + [0])
    data = bytearray(end)
    for off, (_, _, _, raw) in zip(offs, tensors):
        data[off:off + len(raw)] = raw
    return head + b"\0" * (data0 - len(head)) + bytes(data), data0, offs


def t3_head_file(blocks, wtype, n_embd, bias, *, stop=6562, start=6561, vocab=None,
                 extra_kvs=(), extra_tensors=(), **kw):
    """A T3-like GGUF holding the speech_head (raw blocks of ggml type wtype),
    its bias (float32 or None) and the chatterbox.* keys, among other keys and
    tensors of the shapes a T3 file has."""
    n_vocab = len(bias) if bias is not None else (vocab or 0)
    kvs = [("general.architecture", STRING, "chatterbox"),
           ("chatterbox.n_ctx", U32, 8196), ("chatterbox.n_embd", U32, n_embd),
           ("chatterbox.n_head", U32, 16), ("chatterbox.n_layer", U32, 24),
           ("chatterbox.text_vocab_size", U32, 50276),
           ("chatterbox.speech_vocab_size", U32, n_vocab if vocab is None else vocab),
           ("chatterbox.start_speech_token", U32, start),
           ("chatterbox.stop_speech_token", U32, stop),
           ("tokenizer.ggml.tokens", ARRAY, (STRING, ["a", "bc", "", "été"] * 5)),
           ("tokenizer.ggml.scores", ARRAY, (F32, [0.5, -1.0, 2.0])),
           ("misc.flags", ARRAY, (BOOL, [True, False, True])),
           ("misc.i16", I16, -5), ("misc.f64", F64, 2.5), ("misc.u64", U64, 1 << 40),
           ("misc.empty", ARRAY, (U8, []))] + list(extra_kvs)
    raw = np.ascontiguousarray(blocks).tobytes()
    tensors = [("model/wte", (n_embd, 7), GGML_F32, np.zeros((7, n_embd), np.float32).tobytes()),
               ("chatterbox/speech_head", (n_embd, n_vocab), wtype, raw)]
    if bias is not None:
        tensors.append(("chatterbox/speech_head_bias", (n_vocab,), GGML_F32,
                        np.asarray(bias, np.float32).tobytes()))
    tensors += list(extra_tensors)
    return build(kvs, tensors, **kw)
