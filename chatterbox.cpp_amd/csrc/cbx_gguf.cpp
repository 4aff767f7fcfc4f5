// cbx_gguf.cpp -- cbx_gguf_read_head / cbx_gguf_load_head (include/cbx_gguf.h).
//
// The reference reads the T3 GGUF through ggml's gguf reader
// (src/main.cpp:356-399) and takes from it the keys of
// src/chatterbox_t3_internal.h:33-40 and the tensors chatterbox/speech_head and
// chatterbox/speech_head_bias (main.cpp:394-395), as
// scripts/convert-t3-turbo-to-gguf.py:65-104, :160-163, :217-224 writes them.
// This reader walks the file once with a bounded cursor: every length, count
// and offset is checked against the bytes left in the file before it is
// used, so a damaged file fails with CBX_ERR_INVALID instead of reading past
// its end or allocating what its fields claim.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/cbx_gguf.h"
#include "cbx_internal.h"

namespace {

// GGUF value types (ggml's published format)
enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};
// ggml tensor types this reader sizes (the head's formats and the bias's)
enum : uint32_t { kTF32 = 0, kTF16 = 1, kTQ4_0 = 2, kTQ8_0 = 8 };
constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr int kMaxDims = 4;

struct Reader {
    FILE* f = nullptr;
    uint64_t size = 0, pos = 0;
    bool bad = false;
    ~Reader() {
        if (f) fclose(f);
    }
    uint64_t left() const { return size - pos; }
    bool read(void* dst, uint64_t n) {
        if (bad || n > left() || fread(dst, 1, (size_t)n, f) != (size_t)n) {
            bad = true;
            return false;
        }
        pos += n;
        return true;
    }
    bool skip(uint64_t n) {
        if (bad || n > left() || fseeko(f, (off_t)n, SEEK_CUR) != 0) {
            bad = true;
            return false;
        }
        pos += n;
        return true;
    }
    bool u32(uint32_t& v) { return read(&v, 4); }
    bool u64(uint64_t& v) { return read(&v, 8); }
    // a GGUF string: u64 length, then the bytes; kept when keep != nullptr
    bool str(std::string* keep) {
        uint64_t n = 0;
        if (!u64(n) || n > left()) return bad = true, false;
        if (!keep) return skip(n);
        keep->resize((size_t)n);
        return n == 0 || read(&(*keep)[0], n);
    }
};

uint64_t scalar_size(uint32_t t) {
    switch (t) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

// bytes of a tensor of type t with ne[0] = n0 and n_rows rows; 0 if the type
// is not one this reader sizes or n0 does not fill whole blocks
uint64_t tensor_bytes(uint32_t t, uint64_t n0, uint64_t n_rows) {
    switch (t) {
        case kTF32: return 4 * n0 * n_rows;
        case kTF16: return 2 * n0 * n_rows;
        case kTQ4_0: return n0 % 32 ? 0 : 18 * (n0 / 32) * n_rows;
        case kTQ8_0: return n0 % 32 ? 0 : 34 * (n0 / 32) * n_rows;
        default: return 0;
    }
}

struct TensorInfo {
    bool found = false;
    uint32_t n_dims = 0, type = 0;
    uint64_t ne[kMaxDims] = {1, 1, 1, 1};
    uint64_t offset = 0;  // relative to the data section
};

int invalid(const char* path, const char* what) {
    return cbx::set_error(CBX_ERR_INVALID, "cbx_gguf_read_head: %s: %s", path, what);
}

int parse(const char* path, cbx_head_file* out) {
    Reader r;
    r.f = fopen(path, "rb");
    if (!r.f) return cbx::set_error(CBX_ERR_INVALID, "cbx_gguf_read_head: cannot open %s", path);
    if (fseeko(r.f, 0, SEEK_END) != 0) return invalid(path, "cannot seek");
    const off_t end = ftello(r.f);
    if (end < 0 || fseeko(r.f, 0, SEEK_SET) != 0) return invalid(path, "cannot seek");
    r.size = (uint64_t)end;

    uint32_t magic = 0, version = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.u32(magic) || magic != kMagic) return invalid(path, "not a GGUF file (magic)");
    if (!r.u32(version)) return invalid(path, "truncated header");
    if (version != 2 && version != 3)
        return cbx::set_error(CBX_ERR_UNSUPPORTED, "cbx_gguf_read_head: %s: GGUF version %u (2 or 3 supported)",
                              path, version);
    if (!r.u64(n_tensors) || !r.u64(n_kv)) return invalid(path, "truncated header");
    // every pair and tensor info takes at least 12 / 24 bytes of the file
    if (n_kv > r.left() / 12 || n_tensors > r.left() / 24)
        return invalid(path, "counts exceed the file size");

    uint64_t alignment = 32;
    int64_t kv_embd = -1, kv_vocab = -1, kv_start = -1, kv_stop = -1;
    std::string key;
    for (uint64_t i = 0; i < n_kv; ++i) {
        uint32_t type = 0;
        if (!r.str(&key) || !r.u32(type)) return invalid(path, "truncated key/value pair");
        int64_t* want = nullptr;
        if (key == "chatterbox.n_embd") want = &kv_embd;
        else if (key == "chatterbox.speech_vocab_size") want = &kv_vocab;
        else if (key == "chatterbox.start_speech_token") want = &kv_start;
        else if (key == "chatterbox.stop_speech_token") want = &kv_stop;
        const bool is_align = key == "general.alignment";
        if (want || is_align) {
            if (type != kU32 && type != kI32)
                return invalid(path, (key + " is not a 32-bit integer").c_str());
            uint32_t v = 0;
            if (!r.u32(v)) return invalid(path, "truncated value");
            if (is_align) {
                if (type != kU32 || v == 0 || (v & (v - 1)) != 0)
                    return invalid(path, "general.alignment is not a power of two");
                alignment = v;
            } else {
                if (type == kI32 && (int32_t)v < 0) return invalid(path, (key + " is negative").c_str());
                if (v > 0x7fffffffu) return invalid(path, (key + " out of range").c_str());
                *want = (int64_t)v;
            }
            continue;
        }
        if (type == kString) {
            if (!r.str(nullptr)) return invalid(path, "truncated string value");
        } else if (type == kArray) {
            uint32_t et = 0;
            uint64_t count = 0;
            if (!r.u32(et) || !r.u64(count)) return invalid(path, "truncated array");
            if (et == kString) {
                if (count > r.left() / 8) return invalid(path, "array exceeds the file size");
                for (uint64_t j = 0; j < count; ++j)
                    if (!r.str(nullptr)) return invalid(path, "truncated string array");
            } else {
                const uint64_t es = scalar_size(et);
                if (es == 0) return invalid(path, "array of an unknown or nested type");
                if (count > r.left() / es) return invalid(path, "array exceeds the file size");
                if (!r.skip(count * es)) return invalid(path, "truncated array");
            }
        } else {
            const uint64_t es = scalar_size(type);
            if (es == 0) return invalid(path, "value of an unknown type");
            if (!r.skip(es)) return invalid(path, "truncated value");
        }
    }

    TensorInfo head, bias;
    std::string name;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo t;
        if (!r.str(&name) || !r.u32(t.n_dims)) return invalid(path, "truncated tensor info");
        if (t.n_dims < 1 || t.n_dims > kMaxDims) return invalid(path, "tensor with 0 or more than 4 dimensions");
        for (uint32_t d = 0; d < t.n_dims; ++d)
            if (!r.u64(t.ne[d])) return invalid(path, "truncated tensor info");
        if (!r.u32(t.type) || !r.u64(t.offset)) return invalid(path, "truncated tensor info");
        t.found = true;
        TensorInfo* slot = name == "chatterbox/speech_head"        ? &head
                           : name == "chatterbox/speech_head_bias" ? &bias
                                                                   : nullptr;
        if (slot) {
            if (slot->found) return invalid(path, ("tensor " + name + " appears twice").c_str());
            *slot = t;
        }
    }
    // the data section starts at the next multiple of the alignment
    const uint64_t data0 = (r.pos + alignment - 1) / alignment * alignment;
    if (data0 > r.size) return invalid(path, "no data section");

    if (!head.found) return invalid(path, "no tensor chatterbox/speech_head");
    int32_t wtype;
    switch (head.type) {
        case kTF16: wtype = CBX_WTYPE_F16; break;
        case kTQ4_0: wtype = CBX_WTYPE_Q4_0; break;
        case kTQ8_0: wtype = CBX_WTYPE_Q8_0; break;
        default:
            return cbx::set_error(CBX_ERR_UNSUPPORTED,
                                  "cbx_gguf_read_head: %s: speech_head has ggml type %u "
                                  "(F16, Q4_0 and Q8_0 are supported)",
                                  path, head.type);
    }
    if (head.n_dims != 2) return invalid(path, "speech_head is not 2-D");
    const uint64_t n_embd = head.ne[0], n_vocab = head.ne[1];
    if (n_embd < 32 || n_embd > 16384 || n_embd % 32)
        return invalid(path, "speech_head n_embd is not a multiple of 32 in 32..16384");
    if (n_vocab < 1 || n_vocab > (uint64_t)cbx::kMaxVocab)
        return invalid(path, "speech_head n_vocab out of range");
    if (kv_embd >= 0 && (uint64_t)kv_embd != n_embd)
        return invalid(path, "chatterbox.n_embd differs from the speech_head's");
    if (kv_vocab >= 0 && (uint64_t)kv_vocab != n_vocab)
        return invalid(path, "chatterbox.speech_vocab_size differs from the speech_head's rows");
    if (kv_stop >= (int64_t)n_vocab) return invalid(path, "stop_speech_token is not a speech id");
    if (head.offset % alignment) return invalid(path, "speech_head data is not aligned");
    const uint64_t wbytes = tensor_bytes(head.type, n_embd, n_vocab);
    if (head.offset > r.size - data0 || wbytes > r.size - data0 - head.offset)
        return invalid(path, "speech_head data runs past the end of the file");

    uint64_t boff = 0, bbytes = 0;
    if (bias.found) {
        if (bias.type != kTF32) return invalid(path, "speech_head_bias is not F32");
        bool column = bias.ne[0] == n_vocab;  // [n_vocab] or [n_vocab, 1, ...]
        for (uint32_t d = 1; d < bias.n_dims; ++d) column = column && bias.ne[d] == 1;
        if (!column) return invalid(path, "speech_head_bias does not hold n_vocab values");
        if (bias.offset % alignment) return invalid(path, "speech_head_bias data is not aligned");
        bbytes = 4 * n_vocab;
        if (bias.offset > r.size - data0 || bbytes > r.size - data0 - bias.offset)
            return invalid(path, "speech_head_bias data runs past the end of the file");
        boff = data0 + bias.offset;
    }

    cbx_head_file o;
    memset(&o, 0, sizeof(o));
    o.n_vocab = (int32_t)n_vocab;
    o.n_embd = (int32_t)n_embd;
    o.wtype = wtype;
    o.has_bias = bias.found ? 1 : 0;
    o.speech_vocab_size = (int32_t)kv_vocab;
    o.start_speech_token = (int32_t)kv_start;
    o.stop_speech_token = (int32_t)kv_stop;
    o.gguf_version = (int32_t)version;
    o.weight_offset = data0 + head.offset;
    o.weight_bytes = wbytes;
    o.bias_offset = boff;
    o.bias_bytes = bbytes;
    *out = o;
    return CBX_OK;
}

// bytes [off, off + n) of the file into device memory at dst, through a
// host buffer of at most 8 MB
int copy_to_device(const char* path, uint64_t off, uint64_t n, void* dst) {
    FILE* f = fopen(path, "rb");
    if (!f) return cbx::set_error(CBX_ERR_INVALID, "cbx_gguf_load_head: cannot open %s", path);
    std::vector<unsigned char> buf;
    try {
        buf.resize((size_t)(n < (8u << 20) ? n : (8u << 20)));
    } catch (...) {
        fclose(f);
        return cbx::set_error(CBX_ERR_NOMEM, "cbx_gguf_load_head: host buffer");
    }
    int rc = CBX_OK;
    if (fseeko(f, (off_t)off, SEEK_SET) != 0)
        rc = cbx::set_error(CBX_ERR_INVALID, "cbx_gguf_load_head: %s: cannot seek", path);
    for (uint64_t done = 0; rc == CBX_OK && done < n;) {
        const size_t c = (size_t)(n - done < buf.size() ? n - done : buf.size());
        if (fread(buf.data(), 1, c, f) != c) {
            rc = cbx::set_error(CBX_ERR_INVALID, "cbx_gguf_load_head: %s: short read", path);
            break;
        }
        const hipError_t e = hipMemcpy((unsigned char*)dst + done, buf.data(), c, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            rc = cbx::set_error(CBX_ERR_HIP, "cbx_gguf_load_head: hipMemcpy: %s", hipGetErrorString(e));
            break;
        }
        done += c;
    }
    fclose(f);
    return rc;
}

}  // namespace

extern "C" int cbx_gguf_read_head(const char* path, cbx_head_file* out) {
    if (!path || !out) return cbx::set_error(CBX_ERR_INVALID, "cbx_gguf_read_head: NULL argument");
    try {
        return parse(path, out);
    } catch (...) {
        return cbx::set_error(CBX_ERR_NOMEM, "cbx_gguf_read_head: out of host memory");
    }
}

extern "C" int cbx_gguf_load_head(const char* path, const cbx_head_file* info, void* d_weights,
                                  float* d_bias) {
    if (!path || !info || !d_weights)
        return cbx::set_error(CBX_ERR_INVALID, "cbx_gguf_load_head: NULL argument");
    cbx_head_file now;
    const int rc = cbx_gguf_read_head(path, &now);
    if (rc != CBX_OK) return rc;
    if (memcmp(&now, info, sizeof(now)) != 0)
        return cbx::set_error(CBX_ERR_INVALID,
                              "cbx_gguf_load_head: %s does not match the info passed (changed since read?)",
                              path);
    int e = copy_to_device(path, now.weight_offset, now.weight_bytes, d_weights);
    if (e == CBX_OK && now.has_bias && d_bias)
        e = copy_to_device(path, now.bias_offset, now.bias_bytes, d_bias);
    return e;
}
