// cbx_gguf.cpp -- cbx_gguf_read_head / cbx_gguf_load_head and
// cbx_gguf_read_t3 / cbx_gguf_load_t3 (include/cbx_gguf.h).
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
#include <map>
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
enum : uint32_t { kTF32 = 0, kTF16 = 1, kTQ4_0 = 2, kTQ5_0 = 6, kTQ8_0 = 8 };
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
        case kTQ5_0: return n0 % 32 ? 0 : 22 * (n0 / 32) * n_rows;
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

// Everything one walk of a GGUF takes from it: the header, the keys the
// readers use, and every tensor's info by name.
struct Scan {
    uint32_t version = 0;
    uint64_t size = 0, data0 = 0, alignment = 32;
    int64_t kv_embd = -1, kv_vocab = -1, kv_start = -1, kv_stop = -1;
    int64_t kv_ctx = -1, kv_head = -1, kv_layer = -1;
    bool has_eps = false;
    float eps = 0.0f;
    std::map<std::string, TensorInfo> tensors;
    const TensorInfo* find(const std::string& name) const {
        const auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
};

int invalid_in(const char* fn, const char* path, const char* what) {
    return cbx::set_error(CBX_ERR_INVALID, "%s: %s: %s", fn, path, what);
}

// One bounded walk of the file at `path` (fn names the entry point in
// messages): header, key/value pairs, tensor infos.
int scan(const char* fn, const char* path, Scan& s) {
    Reader r;
    r.f = fopen(path, "rb");
    if (!r.f) return cbx::set_error(CBX_ERR_INVALID, "%s: cannot open %s", fn, path);
    auto invalid = [&](const std::string& what) { return invalid_in(fn, path, what.c_str()); };
    if (fseeko(r.f, 0, SEEK_END) != 0) return invalid("cannot seek");
    const off_t end = ftello(r.f);
    if (end < 0 || fseeko(r.f, 0, SEEK_SET) != 0) return invalid("cannot seek");
    r.size = (uint64_t)end;
    s.size = r.size;

    uint32_t magic = 0, version = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.u32(magic) || magic != kMagic) return invalid("not a GGUF file (magic)");
    if (!r.u32(version)) return invalid("truncated header");
    if (version != 2 && version != 3)
        return cbx::set_error(CBX_ERR_UNSUPPORTED, "%s: %s: GGUF version %u (2 or 3 supported)", fn,
                              path, version);
    s.version = version;
    if (!r.u64(n_tensors) || !r.u64(n_kv)) return invalid("truncated header");
    // every pair and tensor info takes at least 12 / 24 bytes of the file
    if (n_kv > r.left() / 12 || n_tensors > r.left() / 24)
        return invalid("counts exceed the file size");

    std::string key;
    for (uint64_t i = 0; i < n_kv; ++i) {
        uint32_t type = 0;
        if (!r.str(&key) || !r.u32(type)) return invalid("truncated key/value pair");
        int64_t* want = nullptr;
        if (key == "chatterbox.n_embd") want = &s.kv_embd;
        else if (key == "chatterbox.speech_vocab_size") want = &s.kv_vocab;
        else if (key == "chatterbox.start_speech_token") want = &s.kv_start;
        else if (key == "chatterbox.stop_speech_token") want = &s.kv_stop;
        else if (key == "chatterbox.n_ctx") want = &s.kv_ctx;
        else if (key == "chatterbox.n_head") want = &s.kv_head;
        else if (key == "chatterbox.n_layer") want = &s.kv_layer;
        const bool is_align = key == "general.alignment";
        if (key == "chatterbox.layer_norm_eps") {
            if (type != kF32) return invalid(key + " is not a 32-bit float");
            if (!r.read(&s.eps, 4)) return invalid("truncated value");
            s.has_eps = true;
            continue;
        }
        if (want || is_align) {
            if (type != kU32 && type != kI32) return invalid(key + " is not a 32-bit integer");
            uint32_t v = 0;
            if (!r.u32(v)) return invalid("truncated value");
            if (is_align) {
                if (type != kU32 || v == 0 || (v & (v - 1)) != 0)
                    return invalid("general.alignment is not a power of two");
                s.alignment = v;
            } else {
                if (type == kI32 && (int32_t)v < 0) return invalid(key + " is negative");
                if (v > 0x7fffffffu) return invalid(key + " out of range");
                *want = (int64_t)v;
            }
            continue;
        }
        if (type == kString) {
            if (!r.str(nullptr)) return invalid("truncated string value");
        } else if (type == kArray) {
            uint32_t et = 0;
            uint64_t count = 0;
            if (!r.u32(et) || !r.u64(count)) return invalid("truncated array");
            if (et == kString) {
                if (count > r.left() / 8) return invalid("array exceeds the file size");
                for (uint64_t j = 0; j < count; ++j)
                    if (!r.str(nullptr)) return invalid("truncated string array");
            } else {
                const uint64_t es = scalar_size(et);
                if (es == 0) return invalid("array of an unknown or nested type");
                if (count > r.left() / es) return invalid("array exceeds the file size");
                if (!r.skip(count * es)) return invalid("truncated array");
            }
        } else {
            const uint64_t es = scalar_size(type);
            if (es == 0) return invalid("value of an unknown type");
            if (!r.skip(es)) return invalid("truncated value");
        }
    }

    std::string name;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo t;
        if (!r.str(&name) || !r.u32(t.n_dims)) return invalid("truncated tensor info");
        if (t.n_dims < 1 || t.n_dims > kMaxDims) return invalid("tensor with 0 or more than 4 dimensions");
        for (uint32_t d = 0; d < t.n_dims; ++d)
            if (!r.u64(t.ne[d])) return invalid("truncated tensor info");
        if (!r.u32(t.type) || !r.u64(t.offset)) return invalid("truncated tensor info");
        t.found = true;
        if (!s.tensors.emplace(name, t).second) return invalid("tensor " + name + " appears twice");
    }
    // the data section starts at the next multiple of the alignment
    s.data0 = (r.pos + s.alignment - 1) / s.alignment * s.alignment;
    if (s.data0 > r.size) return invalid("no data section");
    return CBX_OK;
}

// Whether tensor t's data, `bytes` long, lies aligned inside the data section.
bool data_ok(const Scan& s, const TensorInfo& t, uint64_t bytes) {
    return t.offset % s.alignment == 0 && t.offset <= s.size - s.data0 &&
           bytes <= s.size - s.data0 - t.offset;
}

int parse(const char* path, cbx_head_file* out) {
    const char* fn = "cbx_gguf_read_head";
    Scan s;
    const int rc = scan(fn, path, s);
    if (rc != CBX_OK) return rc;
    auto invalid = [&](const char* what) { return invalid_in(fn, path, what); };
    const TensorInfo* hp = s.find("chatterbox/speech_head");
    const TensorInfo* bp = s.find("chatterbox/speech_head_bias");
    if (!hp) return invalid("no tensor chatterbox/speech_head");
    const TensorInfo& head = *hp;
    int32_t wtype;
    switch (head.type) {
        case kTF16: wtype = CBX_WTYPE_F16; break;
        case kTQ4_0: wtype = CBX_WTYPE_Q4_0; break;
        case kTQ5_0: wtype = CBX_WTYPE_Q5_0; break;
        case kTQ8_0: wtype = CBX_WTYPE_Q8_0; break;
        default:
            return cbx::set_error(CBX_ERR_UNSUPPORTED,
                                  "cbx_gguf_read_head: %s: speech_head has ggml type %u "
                                  "(F16, Q4_0, Q5_0 and Q8_0 are supported)",
                                  path, head.type);
    }
    if (head.n_dims != 2) return invalid("speech_head is not 2-D");
    const uint64_t n_embd = head.ne[0], n_vocab = head.ne[1];
    if (n_embd < 32 || n_embd > 16384 || n_embd % 32)
        return invalid("speech_head n_embd is not a multiple of 32 in 32..16384");
    if (n_vocab < 1 || n_vocab > (uint64_t)cbx::kMaxVocab)
        return invalid("speech_head n_vocab out of range");
    if (s.kv_embd >= 0 && (uint64_t)s.kv_embd != n_embd)
        return invalid("chatterbox.n_embd differs from the speech_head's");
    if (s.kv_vocab >= 0 && (uint64_t)s.kv_vocab != n_vocab)
        return invalid("chatterbox.speech_vocab_size differs from the speech_head's rows");
    if (s.kv_stop >= (int64_t)n_vocab) return invalid("stop_speech_token is not a speech id");
    if (head.offset % s.alignment) return invalid("speech_head data is not aligned");
    const uint64_t wbytes = tensor_bytes(head.type, n_embd, n_vocab);
    if (!data_ok(s, head, wbytes)) return invalid("speech_head data runs past the end of the file");

    uint64_t boff = 0, bbytes = 0;
    if (bp) {
        const TensorInfo& bias = *bp;
        if (bias.type != kTF32) return invalid("speech_head_bias is not F32");
        bool column = bias.ne[0] == n_vocab;  // [n_vocab] or [n_vocab, 1, ...]
        for (uint32_t d = 1; d < bias.n_dims; ++d) column = column && bias.ne[d] == 1;
        if (!column) return invalid("speech_head_bias does not hold n_vocab values");
        if (bias.offset % s.alignment) return invalid("speech_head_bias data is not aligned");
        bbytes = 4 * n_vocab;
        if (!data_ok(s, bias, bbytes))
            return invalid("speech_head_bias data runs past the end of the file");
        boff = s.data0 + bias.offset;
    }

    cbx_head_file o;
    memset(&o, 0, sizeof(o));
    o.n_vocab = (int32_t)n_vocab;
    o.n_embd = (int32_t)n_embd;
    o.wtype = wtype;
    o.has_bias = bp ? 1 : 0;
    o.speech_vocab_size = (int32_t)s.kv_vocab;
    o.start_speech_token = (int32_t)s.kv_start;
    o.stop_speech_token = (int32_t)s.kv_stop;
    o.gguf_version = (int32_t)s.version;
    o.weight_offset = s.data0 + head.offset;
    o.weight_bytes = wbytes;
    o.bias_offset = boff;
    o.bias_bytes = bbytes;
    *out = o;
    return CBX_OK;
}

// One T3 tensor's place: its bytes in the file and in the device buffer
// (256-byte aligned), widened from F16 to F32 on the way when `widen`.
struct T3Item {
    uint64_t file_off = 0, file_bytes = 0, dev_off = 0;
    bool widen = false;
};

// The T3 tensors of main.cpp:400-416 (names as the converter writes them,
// scripts/convert-t3-turbo-to-gguf.py:150-189), checked for type and shape,
// and their device layout: wpe, speech_emb, ln_f g and b, then per layer the
// 12 tensors in cbx_t3_layer's order.
int plan_t3(const char* fn, const char* path, cbx_t3_file* out, std::vector<T3Item>* items) {
    Scan s;
    int rc = scan(fn, path, s);
    if (rc != CBX_OK) return rc;
    auto invalid = [&](const std::string& what) { return invalid_in(fn, path, what.c_str()); };
    if (s.kv_embd < 0 || s.kv_head < 0 || s.kv_layer < 0 || s.kv_ctx < 0 || !s.has_eps)
        return invalid("missing chatterbox.n_embd, n_head, n_layer, n_ctx or layer_norm_eps");
    const int64_t n = s.kv_embd;
    if (s.kv_layer < 1 || s.kv_layer > 256 || n > 4096 || s.kv_head > 4096 ||
        !cbx::t3_shape_ok((int32_t)n, (int32_t)s.kv_head))
        return cbx::set_error(CBX_ERR_UNSUPPORTED,
                              "%s: %s: n_layer %lld, n_embd %lld, n_head %lld (1..256 layers, heads "
                              "of 64, n_embd in {256..1024 by 256, 1536, 2048, 3072, 4096})",
                              fn, path, (long long)s.kv_layer, (long long)n, (long long)s.kv_head);
    if (!(s.eps >= 0.0f)) return invalid("layer_norm_eps is negative or NaN");
    std::vector<T3Item> plan;
    uint64_t dev = 0;
    auto add = [&](const std::string& name, uint64_t ne0, uint64_t ne1, bool matrix,
                   uint32_t* mtype, int64_t* rows_out) -> int {
        const TensorInfo* t = s.find(name);
        if (!t) return invalid("no tensor " + name);
        bool shape = t->ne[0] == ne0 && (ne1 == 0 || t->ne[1] == ne1);
        for (uint32_t d = ne1 ? 2 : 1; d < t->n_dims; ++d) shape = shape && t->ne[d] == 1;
        if (rows_out) {  // rows taken from the file (speech_emb, wpe)
            shape = t->ne[0] == ne0 && t->n_dims >= 2 && t->ne[1] >= 1 && t->ne[1] <= 0x7fffffff;
            for (uint32_t d = 2; d < t->n_dims; ++d) shape = shape && t->ne[d] == 1;
        }
        if (!shape) return invalid("tensor " + name + " has the wrong shape");
        const uint64_t rows = rows_out ? t->ne[1] : (ne1 ? ne1 : 1);
        T3Item it;
        if (matrix) {
            if (t->type != kTF16 && t->type != kTQ4_0 && t->type != kTQ5_0 && t->type != kTQ8_0)
                return cbx::set_error(CBX_ERR_UNSUPPORTED, "%s: %s: %s has ggml type %u (F16, Q4_0, "
                                      "Q5_0 and Q8_0 are supported)", fn, path, name.c_str(), t->type);
            if (*mtype == ~0u) *mtype = t->type;
            if (t->type != *mtype)
                return cbx::set_error(CBX_ERR_UNSUPPORTED, "%s: %s: the layer matrices mix ggml types",
                                      fn, path);
            it.file_bytes = tensor_bytes(t->type, ne0, rows);
            if (it.file_bytes == 0) return invalid("tensor " + name + " does not fill whole blocks");
        } else if (t->type == kTF32) {
            it.file_bytes = 4 * ne0 * rows;
        } else if (t->type == kTF16 && rows_out) {  // speech_emb as the converter writes it
            it.file_bytes = 2 * ne0 * rows;
            it.widen = true;
        } else {
            return invalid("tensor " + name + " is not F32");
        }
        if (!data_ok(s, *t, it.file_bytes)) return invalid("tensor " + name + " runs past the end of the file");
        it.file_off = s.data0 + t->offset;
        it.dev_off = dev;
        dev += ((it.widen ? 2 * it.file_bytes : it.file_bytes) + 255) / 256 * 256;
        plan.push_back(it);
        if (rows_out) *rows_out = (int64_t)rows;
        return CBX_OK;
    };
    uint32_t mtype = ~0u;
    int64_t n_pos = 0, n_vocab = 0;
    if ((rc = add("model/wpe", n, 0, false, nullptr, &n_pos)) != CBX_OK) return rc;
    if ((rc = add("chatterbox/speech_emb", n, 0, false, nullptr, &n_vocab)) != CBX_OK) return rc;
    if ((rc = add("model/ln_f/g", n, 0, false, nullptr, nullptr)) != CBX_OK) return rc;
    if ((rc = add("model/ln_f/b", n, 0, false, nullptr, nullptr)) != CBX_OK) return rc;
    if (n_pos != s.kv_ctx) return invalid("model/wpe rows differ from chatterbox.n_ctx");
    if (s.kv_vocab >= 0 && n_vocab != s.kv_vocab)
        return invalid("chatterbox/speech_emb rows differ from chatterbox.speech_vocab_size");
    for (int64_t l = 0; l < s.kv_layer; ++l) {
        const std::string p = "model/h" + std::to_string(l) + "/";
        struct { const char* sfx; uint64_t ne0, ne1; bool m; } const ts[12] = {
            {"ln_1/g", (uint64_t)n, 0, false},          {"ln_1/b", (uint64_t)n, 0, false},
            {"attn/c_attn/w", (uint64_t)n, 3 * (uint64_t)n, true},
            {"attn/c_attn/b", 3 * (uint64_t)n, 0, false},
            {"attn/c_proj/w", (uint64_t)n, (uint64_t)n, true},
            {"attn/c_proj/b", (uint64_t)n, 0, false},   {"ln_2/g", (uint64_t)n, 0, false},
            {"ln_2/b", (uint64_t)n, 0, false},
            {"mlp/c_fc/w", (uint64_t)n, 4 * (uint64_t)n, true},
            {"mlp/c_fc/b", 4 * (uint64_t)n, 0, false},
            {"mlp/c_proj/w", 4 * (uint64_t)n, (uint64_t)n, true},
            {"mlp/c_proj/b", (uint64_t)n, 0, false}};
        for (const auto& e : ts)
            if ((rc = add(p + e.sfx, e.ne0, e.ne1, e.m, &mtype, nullptr)) != CBX_OK) return rc;
    }
    cbx_t3_file o;
    memset(&o, 0, sizeof(o));
    o.n_layer = (int32_t)s.kv_layer;
    o.n_embd = (int32_t)n;
    o.n_head = (int32_t)s.kv_head;
    o.n_pos = (int32_t)n_pos;
    o.n_speech_vocab = (int32_t)n_vocab;
    o.wtype = mtype == kTF16 ? CBX_WTYPE_F16
            : mtype == kTQ4_0 ? CBX_WTYPE_Q4_0
            : mtype == kTQ5_0 ? CBX_WTYPE_Q5_0
                              : CBX_WTYPE_Q8_0;
    o.eps = s.eps;
    o.start_speech_token = (int32_t)s.kv_start;
    o.stop_speech_token = (int32_t)s.kv_stop;
    o.gguf_version = (int32_t)s.version;
    o.device_bytes = dev;
    *out = o;
    if (items) *items = std::move(plan);
    return CBX_OK;
}

// bytes [off, off + n) of the file into device memory at dst, through a
// host buffer of at most 8 MB; widen: the bytes are F16 values, stored as F32
int copy_to_device(const char* fn, const char* path, uint64_t off, uint64_t n, void* dst,
                   bool widen = false) {
    FILE* f = fopen(path, "rb");
    if (!f) return cbx::set_error(CBX_ERR_INVALID, "%s: cannot open %s", fn, path);
    std::vector<unsigned char> buf;
    std::vector<float> wide;
    try {
        buf.resize((size_t)(n < (8u << 20) ? n : (8u << 20)));
        if (widen) wide.resize(buf.size() / 2);
    } catch (...) {
        fclose(f);
        return cbx::set_error(CBX_ERR_NOMEM, "%s: host buffer", fn);
    }
    int rc = CBX_OK;
    if (fseeko(f, (off_t)off, SEEK_SET) != 0)
        rc = cbx::set_error(CBX_ERR_INVALID, "%s: %s: cannot seek", fn, path);
    for (uint64_t done = 0; rc == CBX_OK && done < n;) {
        const size_t c = (size_t)(n - done < buf.size() ? n - done : buf.size());
        if (fread(buf.data(), 1, c, f) != c) {
            rc = cbx::set_error(CBX_ERR_INVALID, "%s: %s: short read", fn, path);
            break;
        }
        hipError_t e;
        if (widen) {  // binary16 -> binary32 is exact
            for (size_t i = 0; i < c / 2; ++i) {
                uint16_t h;
                memcpy(&h, &buf[2 * i], 2);
                wide[i] = (float)__builtin_bit_cast(_Float16, h);
            }
            e = hipMemcpy((unsigned char*)dst + 2 * done, wide.data(), 2 * c, hipMemcpyHostToDevice);
        } else {
            e = hipMemcpy((unsigned char*)dst + done, buf.data(), c, hipMemcpyHostToDevice);
        }
        if (e != hipSuccess) {
            rc = cbx::set_error(CBX_ERR_HIP, "%s: hipMemcpy: %s", fn, hipGetErrorString(e));
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
    const char* fn = "cbx_gguf_load_head";
    int e = copy_to_device(fn, path, now.weight_offset, now.weight_bytes, d_weights);
    if (e == CBX_OK && now.has_bias && d_bias)
        e = copy_to_device(fn, path, now.bias_offset, now.bias_bytes, d_bias);
    return e;
}

extern "C" int cbx_gguf_read_t3(const char* path, cbx_t3_file* out) {
    if (!path || !out) return cbx::set_error(CBX_ERR_INVALID, "cbx_gguf_read_t3: NULL argument");
    try {
        return plan_t3("cbx_gguf_read_t3", path, out, nullptr);
    } catch (...) {
        return cbx::set_error(CBX_ERR_NOMEM, "cbx_gguf_read_t3: out of host memory");
    }
}

extern "C" int cbx_gguf_load_t3(const char* path, const cbx_t3_file* info, void* d_buffer,
                                cbx_t3_layer* layers, cbx_t3_model* model) {
    const char* fn = "cbx_gguf_load_t3";
    if (!path || !info || !d_buffer || !layers || !model)
        return cbx::set_error(CBX_ERR_INVALID, "%s: NULL argument", fn);
    try {
        cbx_t3_file now;
        std::vector<T3Item> items;
        int rc = plan_t3(fn, path, &now, &items);
        if (rc != CBX_OK) return rc;
        if (memcmp(&now, info, sizeof(now)) != 0)
            return cbx::set_error(CBX_ERR_INVALID,
                                  "%s: %s does not match the info passed (changed since read?)", fn,
                                  path);
        for (const T3Item& it : items)
            if ((rc = copy_to_device(fn, path, it.file_off, it.file_bytes,
                                     (unsigned char*)d_buffer + it.dev_off, it.widen)) != CBX_OK)
                return rc;
        auto at = [&](size_t i) { return (void*)((unsigned char*)d_buffer + items[i].dev_off); };
        for (int l = 0; l < now.n_layer; ++l) {
            const size_t b = 4 + 12 * (size_t)l;
            cbx_t3_layer& L = layers[l];
            L.ln_1_g = (const float*)at(b + 0);
            L.ln_1_b = (const float*)at(b + 1);
            L.attn_w = at(b + 2);
            L.attn_b = (const float*)at(b + 3);
            L.attn_proj_w = at(b + 4);
            L.attn_proj_b = (const float*)at(b + 5);
            L.ln_2_g = (const float*)at(b + 6);
            L.ln_2_b = (const float*)at(b + 7);
            L.fc_w = at(b + 8);
            L.fc_b = (const float*)at(b + 9);
            L.fc_proj_w = at(b + 10);
            L.fc_proj_b = (const float*)at(b + 11);
        }
        cbx_t3_model m;
        memset(&m, 0, sizeof(m));
        m.n_layer = now.n_layer;
        m.n_embd = now.n_embd;
        m.n_head = now.n_head;
        m.n_pos = now.n_pos;
        m.n_speech_vocab = now.n_speech_vocab;
        m.wtype = now.wtype;
        m.eps = now.eps;
        m.wpe = (const float*)at(0);
        m.speech_emb = (const float*)at(1);
        m.ln_f_g = (const float*)at(2);
        m.ln_f_b = (const float*)at(3);
        m.layers = layers;
        *model = m;
        return CBX_OK;
    } catch (...) {
        return cbx::set_error(CBX_ERR_NOMEM, "%s: out of host memory", fn);
    }
}
