// Checkpoint readers of libaarambh_hip (host code): the GGUF v1 container that
// aarambh-studio writes (weights/src/gguf.rs) and safetensors checkpoints
// (weights/src/lib.rs:68-99).  Tensors are decoded to f32 exactly as the
// reference decodes them, matched to the context's checkpoint tensors by name
// (model/src/model.rs named_tensors order and names) and uploaded through
// aarh_load_tensor_f32, which quantises them on the device into the context's
// formats (INT4 g128 / INT8 per row / bf16 tiles, or f32).
//
// Built without floating-point contraction: q * scale + min is two roundings,
// as in the reference (gguf_quant.rs:37-49).
#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/aarambh_hip.h"

namespace {

thread_local std::string g_host_err;

// ---------------------------------------------------------------------------
// A small JSON reader (metadata of GGUF v1 and safetensors headers).
// ---------------------------------------------------------------------------
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    std::string str;  // string value, or the literal text of a number
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal* get(const char* key) const {
        if (kind != OBJ) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char* p;
    const char* end;
    int depth = 0;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if ((size_t)(end - p) < n || memcmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    bool str(std::string& out) {
        if (p >= end || *p != '"') return false;
        p++;
        out.clear();
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) return false;
                char e = *p++;
                switch (e) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (end - p < 4) return false;
                        unsigned cp = 0;
                        for (int i = 0; i < 4; i++) {
                            char h = *p++;
                            cp <<= 4;
                            if (h >= '0' && h <= '9') cp |= (unsigned)(h - '0');
                            else if (h >= 'a' && h <= 'f') cp |= (unsigned)(h - 'a' + 10);
                            else if (h >= 'A' && h <= 'F') cp |= (unsigned)(h - 'A' + 10);
                            else return false;
                        }
                        // UTF-8 encode (basic plane; surrogate pairs kept as two code points)
                        if (cp < 0x80) {
                            out += (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xC0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3F));
                        } else {
                            out += (char)(0xE0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3F));
                            out += (char)(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: return false;
                }
            } else {
                out += c;
            }
        }
        if (p >= end) return false;
        p++;
        return true;
    }
    bool value(JVal& v) {
        if (++depth > 64) return false;
        ws();
        if (p >= end) return false;
        bool ok = true;
        if (*p == '{') {
            p++;
            v.kind = JVal::OBJ;
            ws();
            if (p < end && *p == '}') {
                p++;
            } else {
                for (;;) {
                    ws();
                    std::pair<std::string, JVal> kv;
                    if (!str(kv.first)) return false;
                    ws();
                    if (p >= end || *p != ':') return false;
                    p++;
                    if (!value(kv.second)) return false;
                    v.obj.push_back(std::move(kv));
                    ws();
                    if (p < end && *p == ',') { p++; continue; }
                    if (p < end && *p == '}') { p++; break; }
                    return false;
                }
            }
        } else if (*p == '[') {
            p++;
            v.kind = JVal::ARR;
            ws();
            if (p < end && *p == ']') {
                p++;
            } else {
                for (;;) {
                    JVal e;
                    if (!value(e)) return false;
                    v.arr.push_back(std::move(e));
                    ws();
                    if (p < end && *p == ',') { p++; continue; }
                    if (p < end && *p == ']') { p++; break; }
                    return false;
                }
            }
        } else if (*p == '"') {
            v.kind = JVal::STR;
            ok = str(v.str);
        } else if (lit("true")) {
            v.kind = JVal::BOOL;
            v.b = true;
        } else if (lit("false")) {
            v.kind = JVal::BOOL;
        } else if (lit("null")) {
            v.kind = JVal::NUL;
        } else {
            const char* s = p;
            while (p < end && *p != '\0' && strchr("+-0123456789.eE", *p) != nullptr) p++;
            if (p == s) return false;
            v.kind = JVal::NUM;
            v.str.assign(s, p);
            char* e = nullptr;
            v.num = strtod(v.str.c_str(), &e);
            ok = e && *e == '\0';
        }
        depth--;
        return ok;
    }
};

bool parse_json(const std::string& text, JVal& out) {
    JParser ps{text.data(), text.data() + text.size()};
    if (!ps.value(out)) return false;
    ps.ws();
    return ps.p == ps.end;
}

bool json_i64(const JVal* v, int64_t* out) {
    if (!v || v->kind != JVal::NUM) return false;
    char* e = nullptr;
    errno = 0;
    long long x = strtoll(v->str.c_str(), &e, 10);
    if (errno || !e || *e != '\0') return false;
    *out = (int64_t)x;
    return true;
}

// ---------------------------------------------------------------------------
// Reference codecs (quant/src/gguf_quant.rs, dequant.rs)
// ---------------------------------------------------------------------------
// f16_to_f32, gguf_quant.rs:86-112
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1F;
    uint32_t mant = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -14;
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                e--;
            }
            mant &= 0x3FFu;
            bits = sign | ((uint32_t)(e + 127) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

constexpr int Q4KM_BLOCK = 256;  // gguf_quant.rs:2
constexpr int Q4KM_BYTES = 132;  // gguf_quant.rs:4
enum { ENC_F32 = 0, ENC_Q8_0 = 1, ENC_Q4KM = 2 };  // TensorEncoding, gguf.rs:24-29

// decode_tensor (gguf.rs:143-241): payload -> n f32 values.
bool decode_payload(int enc, const std::vector<uint8_t>& pl, int64_t n, float* out, std::string& err) {
    if (enc == ENC_F32) {
        if (pl.size() % 4 || (int64_t)(pl.size() / 4) != n) {
            err = "invalid F32 GGUF payload length";
            return false;
        }
        memcpy(out, pl.data(), pl.size());
        return true;
    }
    if (enc == ENC_Q8_0) {
        if (pl.size() < 4 || (int64_t)(pl.size() - 4) != n) {
            err = "invalid Q8_0 payload";
            return false;
        }
        float scale;
        memcpy(&scale, pl.data(), 4);
        for (int64_t i = 0; i < n; i++) out[i] = (float)(int8_t)pl[4 + i] * scale;
        return true;
    }
    if (enc == ENC_Q4KM) {
        if (pl.size() % Q4KM_BYTES) {
            err = "invalid Q4_K_M GGUF payload length";
            return false;
        }
        const int64_t nb = (int64_t)(pl.size() / Q4KM_BYTES);
        if (nb * Q4KM_BLOCK < n) {
            err = "Q4_K_M payload holds fewer values than its shape";
            return false;
        }
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t* blk = pl.data() + b * Q4KM_BYTES;
            const float scale = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            const float mn = f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
            for (int i = 0; i < Q4KM_BLOCK / 2; i++) {
                const int64_t j = b * Q4KM_BLOCK + 2 * i;
                const uint8_t byte = blk[4 + i];
                const float p0 = (float)(byte & 0x0F) * scale;
                const float p1 = (float)(byte >> 4) * scale;
                if (j < n) out[j] = p0 + mn;
                if (j + 1 < n) out[j + 1] = p1 + mn;
            }
        }
        return true;
    }
    err = "unknown GGUF tensor encoding " + std::to_string(enc);
    return false;
}

int64_t numel(const std::vector<int64_t>& shape);
bool payload_fits(int enc, uint64_t len, int64_t n);

// ---------------------------------------------------------------------------
// GGUF v1 reader (load_gguf_tensors, gguf.rs:91-125)
// ---------------------------------------------------------------------------
struct File {
    FILE* f = nullptr;
    ~File() {
        if (f) fclose(f);
    }
};

struct GgufTensor {
    std::string name;
    std::vector<int64_t> shape;
    int enc = 0;
    uint64_t payload_len = 0;
    long payload_off = 0;
};

struct Gguf {
    File file;
    JVal meta;
    std::vector<GgufTensor> tensors;
};

bool rd(FILE* f, void* p, size_t n) { return fread(p, 1, n, f) == n; }
bool rd_u64(FILE* f, uint64_t* v) { return rd(f, v, 8); }

// Reads the header and the tensor index (payloads are read on demand).
int gguf_open(const char* path, Gguf& g, std::string& err) {
    g.file.f = fopen(path, "rb");
    if (!g.file.f) {
        err = std::string("cannot open ") + path + ": " + strerror(errno);
        return AARH_ERR_IO;
    }
    FILE* f = g.file.f;
    fseek(f, 0, SEEK_END);
    const uint64_t fsize = (uint64_t)ftell(f);
    fseek(f, 0, SEEK_SET);
    char magic[4];
    uint32_t version = 0;
    if (!rd(f, magic, 4) || memcmp(magic, "GGUF", 4) != 0) {
        err = std::string(path) + " is not an Aarambh GGUF file";
        return AARH_ERR_CHECKPOINT;
    }
    if (!rd(f, &version, 4) || version != 1) {
        err = "unsupported GGUF version " + std::to_string(version) + ", expected 1";
        return AARH_ERR_CHECKPOINT;
    }
    uint64_t mlen = 0;
    if (!rd_u64(f, &mlen) || mlen > (1u << 26) || mlen > fsize) {
        err = "invalid GGUF metadata length";
        return AARH_ERR_CHECKPOINT;
    }
    std::string meta(mlen, '\0');
    if (!rd(f, &meta[0], mlen) || !parse_json(meta, g.meta) || g.meta.kind != JVal::OBJ) {
        err = "invalid GGUF metadata JSON";
        return AARH_ERR_CHECKPOINT;
    }
    uint64_t count = 0;
    if (!rd_u64(f, &count) || count > (1u << 24)) {
        err = "invalid GGUF tensor count";
        return AARH_ERR_CHECKPOINT;
    }
    for (uint64_t i = 0; i < count; i++) {
        GgufTensor t;
        uint64_t nl = 0, nd = 0;
        if (!rd_u64(f, &nl) || nl > 4096) { err = "invalid GGUF tensor name"; return AARH_ERR_CHECKPOINT; }
        t.name.resize(nl);
        if (nl && !rd(f, &t.name[0], nl)) { err = "truncated GGUF tensor name"; return AARH_ERR_IO; }
        if (!rd_u64(f, &nd) || nd > 8) { err = "invalid GGUF tensor rank in " + t.name; return AARH_ERR_CHECKPOINT; }
        for (uint64_t d = 0; d < nd; d++) {
            uint64_t dim = 0;
            if (!rd_u64(f, &dim) || dim > (1ull << 40)) { err = "invalid GGUF shape in " + t.name; return AARH_ERR_CHECKPOINT; }
            t.shape.push_back((int64_t)dim);
        }
        uint8_t enc = 0;
        if (!rd(f, &enc, 1)) { err = "truncated GGUF tensor " + t.name; return AARH_ERR_IO; }
        if (enc > ENC_Q4KM) { err = "unknown GGUF tensor encoding " + std::to_string(enc); return AARH_ERR_CHECKPOINT; }
        t.enc = enc;
        if (!rd_u64(f, &t.payload_len)) { err = "truncated GGUF tensor " + t.name; return AARH_ERR_IO; }
        t.payload_off = ftell(f);
        if (t.payload_len > fsize - (uint64_t)t.payload_off) { err = "truncated GGUF payload of " + t.name; return AARH_ERR_IO; }
        if (numel(t.shape) < 0) { err = "invalid GGUF shape in " + t.name; return AARH_ERR_CHECKPOINT; }
        if (!payload_fits(t.enc, t.payload_len, numel(t.shape))) {
            err = std::string(t.enc == ENC_F32 ? "invalid F32 GGUF payload length" : t.enc == ENC_Q8_0 ? "invalid Q8_0 payload"
                                                                                   : "invalid Q4_K_M GGUF payload length") +
                  " (" + t.name + ")";
            return AARH_ERR_CHECKPOINT;
        }
        if (fseek(f, (long)t.payload_len, SEEK_CUR) != 0) { err = "truncated GGUF payload of " + t.name; return AARH_ERR_IO; }
        g.tensors.push_back(std::move(t));
    }
    return 0;
}

// Element count of a shape; -1 when it overflows or exceeds 2^40 values (a corrupt header).
int64_t numel(const std::vector<int64_t>& shape) {
    int64_t n = 1;
    for (int64_t d : shape)
        if (d < 0 || __builtin_mul_overflow(n, d, &n) || n > ((int64_t)1 << 40)) return -1;
    return n;
}

// Payload length consistent with the tensor's value count for its encoding
// (decode_f32_tensor / decode_q8_tensor / decode_q4_k_m_tensor, gguf.rs:155-241).
bool payload_fits(int enc, uint64_t len, int64_t n) {
    if (n < 0) return false;
    if (enc == ENC_F32) return len % 4 == 0 && len / 4 == (uint64_t)n;
    if (enc == ENC_Q8_0) return len >= 4 && len - 4 == (uint64_t)n;
    return len % Q4KM_BYTES == 0 && len / Q4KM_BYTES * Q4KM_BLOCK >= (uint64_t)n;
}

int gguf_decode(Gguf& g, const GgufTensor& t, std::vector<float>& out, std::string& err) {
    std::vector<uint8_t> pl(t.payload_len);
    if (fseek(g.file.f, t.payload_off, SEEK_SET) != 0 || (t.payload_len && !rd(g.file.f, pl.data(), t.payload_len))) {
        err = "truncated GGUF payload of " + t.name;
        return AARH_ERR_IO;
    }
    out.assign((size_t)numel(t.shape), 0.f);
    if (!decode_payload(t.enc, pl, (int64_t)out.size(), out.data(), err)) {
        err += " (" + t.name + ")";
        return AARH_ERR_CHECKPOINT;
    }
    return 0;
}

// ---------------------------------------------------------------------------
// safetensors reader
// ---------------------------------------------------------------------------
struct StTensor {
    std::string name, dtype;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
};

int st_open(const char* path, File& file, std::vector<StTensor>& out, uint64_t* data_off, std::string& err) {
    file.f = fopen(path, "rb");
    if (!file.f) {
        err = std::string("cannot open ") + path + ": " + strerror(errno);
        return AARH_ERR_IO;
    }
    fseek(file.f, 0, SEEK_END);
    const uint64_t fsize0 = (uint64_t)ftell(file.f);
    fseek(file.f, 0, SEEK_SET);
    uint64_t hlen = 0;
    if (!rd_u64(file.f, &hlen) || hlen > (1u << 28) || hlen > fsize0) {
        err = "invalid safetensors header length";
        return AARH_ERR_CHECKPOINT;
    }
    std::string h(hlen, '\0');
    JVal root;
    if (!rd(file.f, &h[0], hlen) || !parse_json(h, root) || root.kind != JVal::OBJ) {
        err = "invalid safetensors header JSON";
        return AARH_ERR_CHECKPOINT;
    }
    *data_off = 8 + hlen;
    fseek(file.f, 0, SEEK_END);
    const uint64_t fsize = (uint64_t)ftell(file.f);
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const JVal& v = kv.second;
        StTensor t;
        t.name = kv.first;
        const JVal* dt = v.get("dtype");
        const JVal* sh = v.get("shape");
        const JVal* off = v.get("data_offsets");
        int64_t b = 0, e = 0;
        if (!dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !off || off->kind != JVal::ARR ||
            off->arr.size() != 2 || !json_i64(&off->arr[0], &b) || !json_i64(&off->arr[1], &e) || b < 0 || e < b) {
            err = "invalid safetensors entry " + t.name;
            return AARH_ERR_CHECKPOINT;
        }
        t.dtype = dt->str;
        for (const JVal& d : sh->arr) {
            int64_t x = 0;
            if (!json_i64(&d, &x) || x < 0) {
                err = "invalid safetensors shape of " + t.name;
                return AARH_ERR_CHECKPOINT;
            }
            t.shape.push_back(x);
        }
        t.begin = (uint64_t)b;
        t.end = (uint64_t)e;
        if (*data_off + t.end > fsize) {
            err = "safetensors data of " + t.name + " past the end of the file";
            return AARH_ERR_CHECKPOINT;
        }
        const int64_t n = numel(t.shape);
        const int esz = t.dtype == "F32" ? 4 : (t.dtype == "F16" || t.dtype == "BF16") ? 2 : 0;
        if (n < 0 || (esz && (uint64_t)(t.end - t.begin) != (uint64_t)n * esz)) {
            err = "safetensors byte range of " + t.name + " does not match its shape";
            return AARH_ERR_CHECKPOINT;
        }
        out.push_back(std::move(t));
    }
    return 0;
}

int st_decode(File& file, uint64_t data_off, const StTensor& t, std::vector<float>& out, std::string& err) {
    const int64_t n = numel(t.shape);
    const int esz = t.dtype == "F32" ? 4 : (t.dtype == "F16" || t.dtype == "BF16") ? 2 : 0;
    if (!esz) {
        err = "unsupported safetensors dtype " + t.dtype + " of " + t.name;
        return AARH_ERR_UNSUPPORTED;
    }
    if ((int64_t)(t.end - t.begin) != n * esz) {
        err = "safetensors byte range of " + t.name + " does not match its shape";
        return AARH_ERR_CHECKPOINT;
    }
    std::vector<uint8_t> raw(t.end - t.begin);
    if (fseek(file.f, (long)(data_off + t.begin), SEEK_SET) != 0 || (raw.size() && !rd(file.f, raw.data(), raw.size()))) {
        err = "truncated safetensors data of " + t.name;
        return AARH_ERR_IO;
    }
    out.resize((size_t)n);
    if (esz == 4) {
        memcpy(out.data(), raw.data(), raw.size());
    } else if (t.dtype == "F16") {
        for (int64_t i = 0; i < n; i++) out[i] = f16_to_f32((uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8)));
    } else {
        for (int64_t i = 0; i < n; i++) {
            const uint32_t bits = (uint32_t)(raw[2 * i] | (raw[2 * i + 1] << 8)) << 16;
            memcpy(&out[i], &bits, 4);
        }
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Upload by checkpoint name
// ---------------------------------------------------------------------------
struct Slot {
    int id;
    int64_t rows, cols;
    bool loaded = false;
};

// The two context types (dense aarh_ctx, latent aarh_lat_ctx) behind one set of names.
int num_tensors(aarh_ctx* c) { return aarh_num_tensors(c); }
int num_tensors(aarh_lat_ctx* c) { return aarh_lat_num_tensors(c); }
int tensor_info(aarh_ctx* c, int id, char* name, int cap, int64_t* r, int64_t* cc, int32_t* k) {
    return aarh_tensor_info(c, id, name, cap, r, cc, k);
}
int tensor_info(aarh_lat_ctx* c, int id, char* name, int cap, int64_t* r, int64_t* cc, int32_t* k) {
    return aarh_lat_tensor_info(c, id, name, cap, r, cc, k);
}
int load_f32(aarh_ctx* c, int id, const float* v, int64_t n) { return aarh_load_tensor_f32(c, id, v, n); }
int load_f32(aarh_lat_ctx* c, int id, const float* v, int64_t n) { return aarh_lat_load_tensor_f32(c, id, v, n); }

template <class Ctx>
std::map<std::string, Slot> context_slots(Ctx* ctx) {
    std::map<std::string, Slot> m;
    char name[256];
    const int n = num_tensors(ctx);
    for (int id = 0; id < n; id++) {
        int64_t r = 0, c = 0;
        int32_t kind = 0;
        if (tensor_info(ctx, id, name, sizeof(name), &r, &c, &kind) == AARH_OK) m[name] = Slot{id, r, c};
    }
    return m;
}

// Shape check: 2-D tensors match (rows, cols); the context lists 1-D norms as (1, n).
bool shape_matches(const std::vector<int64_t>& shape, const Slot& s) {
    if (shape.size() == 2) return shape[0] == s.rows && shape[1] == s.cols;
    if (shape.size() == 1) return s.rows == 1 && shape[0] == s.cols;
    return false;
}

}  // namespace

// Set by the library's runtimes (runtime.cpp, lat_runtime.cpp): the context's error text;
// the RoPE scaling check of the dense runtime.
namespace aarh {
int ctx_fail(aarh_ctx* c, int code, const char* msg);
int lat_ctx_fail(aarh_lat_ctx* c, int code, const char* msg);
int rope_scaling_check(int head_dim, int max_seq_len, const aarh_rope_scaling* s, std::string& err);
}  // namespace aarh

namespace {

int fail_ctx(aarh_ctx* c, int code, const std::string& msg) {
    if (c) return aarh::ctx_fail(c, code, msg.c_str());
    g_host_err = msg;
    return code;
}
int fail_ctx(aarh_lat_ctx* c, int code, const std::string& msg) {
    if (c) return aarh::lat_ctx_fail(c, code, msg.c_str());
    g_host_err = msg;
    return code;
}

// ModelConfig.rope_scaling (config.rs:19-47, serde(default) per field, method in snake_case)
// into *out; method AARH_ROPE_NONE when the key is absent or null.  Values are checked by
// the table builder (RopeScalingConfig::validate), not here.
int parse_rope_scaling(const JVal* cfg, aarh_rope_scaling* out, std::string& err) {
    *out = aarh_rope_scaling{AARH_ROPE_NONE, 0, 1.0, 32.0, 1.0, 1.0};
    const JVal* rs = cfg->get("rope_scaling");
    if (!rs || rs->kind == JVal::NUL) return 0;
    if (rs->kind != JVal::OBJ) {
        err = "GGUF config rope_scaling is not an object";
        return AARH_ERR_CHECKPOINT;
    }
    out->method = AARH_ROPE_YARN;
    if (const JVal* m = rs->get("method")) {
        if (m->kind != JVal::STR || (m->str != "yarn" && m->str != "ntk" && m->str != "linear")) {
            err = "GGUF config rope_scaling.method must be \"yarn\", \"ntk\" or \"linear\"";
            return AARH_ERR_CHECKPOINT;
        }
        out->method = m->str == "yarn" ? AARH_ROPE_YARN : m->str == "ntk" ? AARH_ROPE_NTK : AARH_ROPE_LINEAR;
    }
    const struct {
        const char* key;
        double* dst;
    } reals[] = {{"factor", &out->factor},
                 {"beta_fast", &out->beta_fast},
                 {"beta_slow", &out->beta_slow},
                 {"attn_factor", &out->attn_factor}};
    for (const auto& f : reals) {
        const JVal* v = rs->get(f.key);
        if (!v) continue;
        if (v->kind != JVal::NUM) {
            err = std::string("GGUF config rope_scaling.") + f.key + " is not a number";
            return AARH_ERR_CHECKPOINT;
        }
        *f.dst = v->num;
    }
    if (const JVal* v = rs->get("original_max_seq_len")) {
        int64_t n = 0;
        if (!json_i64(v, &n) || n < 0 || n > INT32_MAX) {
            err = "GGUF config rope_scaling.original_max_seq_len is not a valid length";
            return AARH_ERR_CHECKPOINT;
        }
        out->original_max_seq_len = (int32_t)n;
    }
    return 0;
}

// GGUF metadata ModelConfig (core/src/config.rs:732-776) against the context's configuration.
int check_gguf_config(aarh_ctx* c, const JVal& meta) {
    const JVal* cfg = meta.get("config");
    if (!cfg || cfg->kind != JVal::OBJ) return fail_ctx(c, AARH_ERR_CHECKPOINT, "GGUF metadata has no model config");
    aarh_model_config mc{};
    aarh_get_config(c, &mc);
    const struct {
        const char* key;
        int64_t want;
    } fields[] = {{"vocab_size", mc.vocab_size}, {"hidden_dim", mc.hidden_dim}, {"ffn_dim", mc.ffn_dim},
                  {"n_layers", mc.n_layers},     {"n_heads", mc.n_heads},       {"n_kv_heads", mc.n_kv_heads}};
    for (const auto& fld : fields) {
        int64_t v = 0;
        if (!json_i64(cfg->get(fld.key), &v))
            return fail_ctx(c, AARH_ERR_CHECKPOINT, std::string("GGUF config lacks ") + fld.key);
        if (v != fld.want)
            return fail_ctx(c, AARH_ERR_CONFIG, std::string("checkpoint ") + fld.key + " " + std::to_string(v) +
                                                    " does not match the context's " + std::to_string(fld.want));
    }
    const struct {
        const char* key;
        float want;
    } reals[] = {{"rope_theta", mc.rope_theta}, {"norm_eps", mc.norm_eps}};
    for (const auto& fld : reals) {
        const JVal* v = cfg->get(fld.key);
        if (!v || v->kind != JVal::NUM) return fail_ctx(c, AARH_ERR_CHECKPOINT, std::string("GGUF config lacks ") + fld.key);
        if ((float)v->num != fld.want)
            return fail_ctx(c, AARH_ERR_CONFIG, std::string("checkpoint ") + fld.key + " " + v->str +
                                                    " does not match the context's configuration");
    }
    // Layer variants the dense device forward does not implement (latent contexts load them).
    for (const char* key : {"moe", "attention_schedule", "dsa_config"}) {
        const JVal* v = cfg->get(key);
        if (v && v->kind != JVal::NUL)
            return fail_ctx(c, AARH_ERR_UNSUPPORTED, std::string("checkpoint config sets ") + key +
                                                         ", which the dense device forward does not implement");
    }
    const JVal* tie = cfg->get("tie_embeddings");
    if (!tie || tie->kind != JVal::BOOL) return fail_ctx(c, AARH_ERR_CHECKPOINT, "GGUF config lacks tie_embeddings");
    if (tie->b == (mc.untied_lm_head != 0))
        return fail_ctx(c, AARH_ERR_CONFIG, std::string("checkpoint tie_embeddings ") + (tie->b ? "true" : "false") +
                                                " does not match the context's LM head (" +
                                                (mc.untied_lm_head ? "untied" : "tied") + ")");
    // the checkpoint's RoPE (scaled or not) replaces the context's tables
    aarh_rope_scaling rs;
    std::string err;
    int r = parse_rope_scaling(cfg, &rs, err);
    if (r) return fail_ctx(c, r, err);
    return aarh_set_rope_scaling(c, &rs);
}

// Unsigned integer field with a serde default: absent -> def; present and not a valid
// non-negative integer -> false.
bool opt_u32(const JVal* obj, const char* key, int64_t def, int64_t* out) {
    const JVal* v = obj ? obj->get(key) : nullptr;
    if (!v) {
        *out = def;
        return true;
    }
    return json_i64(v, out) && *out >= 0 && *out <= INT32_MAX;
}

// ModelConfig of an MLA + MoE checkpoint (config.rs:732-776) -> the latent context's shape
// fields, with AarambhModel::validate_config's checks (model.rs:281-344) for the parts the
// latent decoder has: MoeConfig::validate (config.rs:179-211), the attention schedule
// (HybridAttentionSchedule::validate, :680-708, GatedDeltaNetConfig::resolve :470-518),
// MlaConfig::resolve / validate (:558-612), RopeScalingConfig::validate (:52-96), and
// dsa_config (DsaConfig::validate :239-258, then "does not select any sparse attention
// layer", since no layer of an all-MLA schedule is full attention).  The latent context runs
// MLA and MoE in every layer (other layer mixes are UNSUPPORTED), with a tied or untied LM
// head as tie_embeddings says.  mtp
// heads, if configured, are not part of the latent context and are ignored (as are qat,
// training-only, model.rs:82-88).  Formats and sizing fields are left as the caller set them.
int lat_config_from_json(const JVal& meta, aarh_lat_config* out, std::string& err) {
    const JVal* cfg = meta.get("config");
    if (!cfg || cfg->kind != JVal::OBJ) {
        err = "GGUF metadata has no model config";
        return AARH_ERR_CHECKPOINT;
    }
    int64_t vocab, hidden, ffn, layers, heads, kv_heads, max_seq;
    const struct {
        const char* key;
        int64_t* dst;
    } ints[] = {{"vocab_size", &vocab}, {"hidden_dim", &hidden}, {"ffn_dim", &ffn},        {"n_layers", &layers},
                {"n_heads", &heads},    {"n_kv_heads", &kv_heads}, {"max_seq_len", &max_seq}};
    for (const auto& f : ints)
        if (!json_i64(cfg->get(f.key), f.dst) || *f.dst < 0 || *f.dst > INT32_MAX) {
            err = std::string("GGUF config lacks a valid ") + f.key;
            return AARH_ERR_CHECKPOINT;
        }
    const JVal* th = cfg->get("rope_theta");
    const JVal* ep = cfg->get("norm_eps");
    const JVal* tie = cfg->get("tie_embeddings");
    if (!th || th->kind != JVal::NUM || !ep || ep->kind != JVal::NUM) {
        err = "GGUF config lacks rope_theta / norm_eps";
        return AARH_ERR_CHECKPOINT;
    }
    if (!tie || tie->kind != JVal::BOOL) {
        err = "GGUF config lacks tie_embeddings";
        return AARH_ERR_CHECKPOINT;
    }
    // validate_config (model.rs:283-313), head_dim == 64 aside (the benchmark shapes differ)
    auto cfg_err = [&](const std::string& m) {
        err = m;
        return AARH_ERR_CONFIG;
    };
    if (vocab == 0) return cfg_err("vocab_size must be non-zero");
    if (hidden == 0 || ffn == 0 || layers == 0) return cfg_err("hidden_dim, ffn_dim, and n_layers must be non-zero");
    if (heads == 0 || kv_heads == 0) return cfg_err("n_heads and n_kv_heads must be non-zero");
    if (max_seq == 0) return cfg_err("max_seq_len must be non-zero");
    if (hidden % heads) return cfg_err("hidden_dim must be divisible by n_heads");
    if (heads % kv_heads) return cfg_err("n_heads must be divisible by n_kv_heads");
    aarh_rope_scaling rs;
    int r = parse_rope_scaling(cfg, &rs, err);
    if (r) return r;
    if (rs.method != AARH_ROPE_NONE && (r = aarh::rope_scaling_check((int)(hidden / heads), (int)max_seq, &rs, err)))
        return r;
    // MoE (moe.validate, config.rs:179-211)
    const JVal* moe = cfg->get("moe");
    if (!moe || moe->kind == JVal::NUL) {
        err = "the latent context runs a MoE FFN in every layer; the checkpoint config has no moe";
        return AARH_ERR_UNSUPPORTED;
    }
    if (moe->kind != JVal::OBJ) {
        err = "GGUF config moe is not an object";
        return AARH_ERR_CHECKPOINT;
    }
    int64_t n_exp, top_k, exp_ffn, every_n, fine, n_shared;
    if (!opt_u32(moe, "num_experts", 8, &n_exp) || !opt_u32(moe, "top_k", 2, &top_k) ||
        !opt_u32(moe, "expert_ffn_dim", 0, &exp_ffn) || !opt_u32(moe, "every_n_layers", 2, &every_n) ||
        !opt_u32(moe, "fine_grained_factor", 1, &fine) || !opt_u32(moe, "num_shared_experts", 0, &n_shared)) {
        err = "GGUF config moe has a field that is not a valid count";
        return AARH_ERR_CHECKPOINT;
    }
    double aux = 0.01;
    if (const JVal* a = moe->get("aux_loss_weight")) {
        if (a->kind != JVal::NUM) {
            err = "GGUF config moe.aux_loss_weight is not a number";
            return AARH_ERR_CHECKPOINT;
        }
        aux = a->num;
    }
    if (n_exp < 2) return cfg_err("moe.num_experts must be at least 2");
    if (fine == 0) return cfg_err("moe.fine_grained_factor must be non-zero");
    if (exp_ffn == 0 || exp_ffn % fine)
        return cfg_err("moe.expert_ffn_dim " + std::to_string(exp_ffn) +
                       " must be non-zero and divisible by fine_grained_factor " + std::to_string(fine));
    const int64_t routed = n_exp * fine;
    if (top_k == 0 || top_k > routed)
        return cfg_err("moe.top_k must be in 1..=" + std::to_string(routed) + " for num_experts=" +
                       std::to_string(n_exp) + " and fine_grained_factor=" + std::to_string(fine));
    if (!(aux >= 0.0) || !std::isfinite(aux)) return cfg_err("moe.aux_loss_weight must be finite and non-negative");
    if (every_n == 0) return cfg_err("moe.every_n_layers must be non-zero");
    if (every_n > layers) return cfg_err("moe.every_n_layers does not select any model layer");
    // what the latent context cannot hold is reported after the reference's own checks
    std::string unsupported;
    if (every_n != 1)
        unsupported = "the latent context runs a MoE FFN in every layer; moe.every_n_layers " +
                      std::to_string(every_n) + " leaves dense FFN layers";
    // attention schedule with MLA in every layer
    const JVal* sch = cfg->get("attention_schedule");
    if (!sch || sch->kind == JVal::NUL) {
        err = "the latent context runs MLA in every layer; the checkpoint config has no attention_schedule";
        return AARH_ERR_UNSUPPORTED;
    }
    if (sch->kind != JVal::OBJ) {
        err = "GGUF config attention_schedule is not an object";
        return AARH_ERR_CHECKPOINT;
    }
    int64_t full_every;
    if (!opt_u32(sch, "full_attention_every_n", 4, &full_every)) {
        err = "GGUF config attention_schedule.full_attention_every_n is not a valid count";
        return AARH_ERR_CHECKPOINT;
    }
    std::vector<bool> is_mla((size_t)layers, false);
    if (const JVal* ml = sch->get("mla_layers")) {
        if (ml->kind != JVal::ARR) {
            err = "GGUF config attention_schedule.mla_layers is not an array";
            return AARH_ERR_CHECKPOINT;
        }
        for (const JVal& v : ml->arr) {
            int64_t l = 0;
            if (!json_i64(&v, &l) || l < 0) {
                err = "GGUF config attention_schedule.mla_layers holds a value that is not a layer index";
                return AARH_ERR_CHECKPOINT;
            }
            if (l < layers) is_mla[(size_t)l] = true;
        }
    }
    if (full_every == 0) return cfg_err("attention_schedule.full_attention_every_n must be non-zero");
    bool all_mla = true, any_mla = false;
    for (bool b : is_mla) all_mla = all_mla && b, any_mla = any_mla || b;
    if (layers < 2 || !any_mla)
        return cfg_err("attention_schedule must select at least one Gated DeltaNet or LatentMLA layer");
    const JVal* mla = sch->get("mla");
    if (!mla || mla->kind == JVal::NUL) return cfg_err("attention_schedule.mla must be set when mla_layers is non-empty");
    if (mla->kind != JVal::OBJ) {
        err = "GGUF config attention_schedule.mla is not an object";
        return AARH_ERR_CHECKPOINT;
    }
    // GatedDeltaNetConfig::resolve + validate run for every schedule (config.rs:707)
    {
        const JVal* gd = sch->get("gated_deltanet");
        if (gd && gd->kind != JVal::OBJ) {
            err = "GGUF config attention_schedule.gated_deltanet is not an object";
            return AARH_ERR_CHECKPOINT;
        }
        int64_t gh, gk, gv, conv, chunk;
        if (!opt_u32(gd, "n_heads", 0, &gh) || !opt_u32(gd, "key_head_dim", 0, &gk) ||
            !opt_u32(gd, "value_head_dim", 0, &gv) || !opt_u32(gd, "conv_kernel_size", 4, &conv) ||
            !opt_u32(gd, "chunk_size", 64, &chunk)) {
            err = "GGUF config attention_schedule.gated_deltanet has a field that is not a valid count";
            return AARH_ERR_CHECKPOINT;
        }
        if (gh == 0) gh = std::max<int64_t>(heads / 2, 1);
        if (gk == 0) gk = hidden * 3 / (4 * gh);
        if (gv == 0) gv = gk * 2;
        if (gh == 0 || gk == 0 || gv == 0)
            return cfg_err("gated_deltanet head counts and dimensions must resolve to non-zero values");
        if (conv < 2) return cfg_err("gated_deltanet.conv_kernel_size must be at least 2");
        if (chunk < 16 || chunk > 256 || (chunk & (chunk - 1)))
            return cfg_err("gated_deltanet.chunk_size must be a power of two in 16..=256");
    }
    if (!all_mla && unsupported.empty())
        unsupported = "the latent context runs MLA in every layer; attention_schedule.mla_layers must list all " +
                      std::to_string(layers) + " layers";
    // MlaConfig::resolve (config.rs:558-587) and validate (:589-612)
    int64_t latent, nope, rope, mheads, vdim;
    if (!opt_u32(mla, "latent_dim", 512, &latent) || !opt_u32(mla, "nope_head_dim", 0, &nope) ||
        !opt_u32(mla, "rope_head_dim", 16, &rope) || !opt_u32(mla, "n_heads", 0, &mheads) ||
        !opt_u32(mla, "value_head_dim", 0, &vdim)) {
        err = "GGUF config attention_schedule.mla has a field that is not a valid count";
        return AARH_ERR_CHECKPOINT;
    }
    if (mheads == 0) mheads = heads;
    if (nope == 0) nope = std::max<int64_t>(hidden / heads > rope ? hidden / heads - rope : 0, 8);
    if (vdim == 0) vdim = nope;
    if (latent == 0) return cfg_err("mla.latent_dim must be non-zero");
    if (mheads == 0) return cfg_err("mla.n_heads must resolve to a non-zero value");
    if (nope == 0) return cfg_err("mla.nope_head_dim must resolve to a non-zero value");
    if (rope == 0 || rope % 2) return cfg_err("mla.rope_head_dim must be a positive even number");
    if (vdim == 0) return cfg_err("mla.value_head_dim must resolve to a non-zero value");
    // dsa_config: validate, then no layer of an all-MLA schedule is a sparse slot
    if (const JVal* dsa = cfg->get("dsa_config"); dsa && dsa->kind != JVal::NUL) {
        int64_t bs, tk, mn;
        if (dsa->kind != JVal::OBJ || !opt_u32(dsa, "block_size", 64, &bs) || !opt_u32(dsa, "top_k_blocks", 16, &tk) ||
            !opt_u32(dsa, "min_seq_len_for_sparsity", 2048, &mn)) {
            err = "GGUF config dsa_config is not a valid object";
            return AARH_ERR_CHECKPOINT;
        }
        if (bs < 16 || bs > 256 || (bs & (bs - 1))) return cfg_err("dsa.block_size must be a power of two in 16..=256");
        if (tk == 0) return cfg_err("dsa.top_k_blocks must be non-zero");
        if (mn < bs) return cfg_err("dsa.min_seq_len_for_sparsity must be at least dsa.block_size");
        // Sparse slots are the schedule's full-attention layers that are not MLA layers
        bool any_sparse = false;
        for (int64_t l = 0; l < layers; l++) any_sparse = any_sparse || (!is_mla[(size_t)l] && l % full_every == 0);
        if (!any_sparse) return cfg_err("dsa_config does not select any sparse attention layer");
    }
    if (!unsupported.empty()) {
        err = unsupported;
        return AARH_ERR_UNSUPPORTED;
    }
    out->untied_lm_head = tie->b ? 0 : 1;  // LmHead::untied_with_qat (model.rs:239-248)
    out->vocab_size = (int32_t)vocab;
    out->hidden_dim = (int32_t)hidden;
    out->n_layers = (int32_t)layers;
    out->n_heads = (int32_t)mheads;
    out->max_seq_len = (int32_t)max_seq;
    out->rope_theta = (float)th->num;
    out->norm_eps = (float)ep->num;
    out->latent_dim = (int32_t)latent;
    out->rope_dim = (int32_t)rope;
    out->nope_dim = (int32_t)nope;
    out->v_dim = (int32_t)vdim;
    out->n_experts = (int32_t)routed;
    out->top_k = (int32_t)top_k;
    out->expert_dim = (int32_t)(exp_ffn / fine);
    out->n_shared = (int32_t)n_shared;
    return 0;
}

// The latent file's shape against the context's (as check_gguf_config for the dense context).
int check_lat_gguf_config(aarh_lat_ctx* c, const JVal& meta) {
    aarh_lat_config want{}, got{};
    aarh_lat_get_config(c, &want);
    std::string err;
    int r = lat_config_from_json(meta, &got, err);
    if (r) return fail_ctx(c, r, err);
    const struct {
        const char* key;
        int32_t file, ctx;
    } f[] = {{"vocab_size", got.vocab_size, want.vocab_size},  {"hidden_dim", got.hidden_dim, want.hidden_dim},
             {"n_layers", got.n_layers, want.n_layers},        {"mla n_heads", got.n_heads, want.n_heads},
             {"mla latent_dim", got.latent_dim, want.latent_dim}, {"mla rope_head_dim", got.rope_dim, want.rope_dim},
             {"mla nope_head_dim", got.nope_dim, want.nope_dim}, {"mla value_head_dim", got.v_dim, want.v_dim},
             {"routed experts", got.n_experts, want.n_experts}, {"moe top_k", got.top_k, want.top_k},
             {"fine expert width", got.expert_dim, want.expert_dim},
             {"moe num_shared_experts", got.n_shared, want.n_shared}};
    for (const auto& x : f)
        if (x.file != x.ctx)
            return fail_ctx(c, AARH_ERR_CONFIG, std::string("checkpoint ") + x.key + " " + std::to_string(x.file) +
                                                    " does not match the context's " + std::to_string(x.ctx));
    if (got.rope_theta != want.rope_theta || got.norm_eps != want.norm_eps)
        return fail_ctx(c, AARH_ERR_CONFIG, "checkpoint rope_theta / norm_eps do not match the context's configuration");
    if (got.untied_lm_head != want.untied_lm_head)
        return fail_ctx(c, AARH_ERR_CONFIG, std::string("checkpoint tie_embeddings ") +
                                                (got.untied_lm_head ? "false" : "true") +
                                                " does not match the context's LM head (" +
                                                (want.untied_lm_head ? "untied" : "tied") + ")");
    return 0;
}

// Every GGUF tensor the context names, decoded and uploaded; every context tensor required.
template <class Ctx>
int load_gguf_into(Ctx* c, Gguf& g, int32_t* out_loaded) {
    auto slots = context_slots(c);
    int loaded = 0, r;
    std::string err;
    std::vector<float> vals;
    for (const GgufTensor& t : g.tensors) {
        auto it = slots.find(t.name);
        if (it == slots.end()) continue;  // tensors of other layer kinds (VarBuilder reads by name)
        if (!shape_matches(t.shape, it->second))
            return fail_ctx(c, AARH_ERR_SHAPE, "checkpoint tensor " + t.name + " has a shape the model does not expect");
        if ((r = gguf_decode(g, t, vals, err))) return fail_ctx(c, r, err);
        if ((r = load_f32(c, it->second.id, vals.data(), (int64_t)vals.size()))) return r;
        it->second.loaded = true;
        loaded++;
    }
    for (const auto& kv : slots)
        if (!kv.second.loaded) return fail_ctx(c, AARH_ERR_CHECKPOINT, "checkpoint lacks tensor " + kv.first);
    if (out_loaded) *out_loaded = loaded;
    return AARH_OK;
}

template <class Ctx>
int load_safetensors_into(Ctx* c, const char* path, int32_t* out_loaded) {
    File file;
    std::vector<StTensor> ts;
    uint64_t data_off = 0;
    std::string err;
    int r = st_open(path, file, ts, &data_off, err);
    if (r) return fail_ctx(c, r, err);
    auto slots = context_slots(c);
    int loaded = 0;
    std::vector<float> vals;
    for (const StTensor& t : ts) {
        auto it = slots.find(t.name);
        if (it == slots.end()) continue;
        if (!shape_matches(t.shape, it->second))
            return fail_ctx(c, AARH_ERR_SHAPE, "checkpoint tensor " + t.name + " has a shape the model does not expect");
        if ((r = st_decode(file, data_off, t, vals, err))) return fail_ctx(c, r, err);
        if ((r = load_f32(c, it->second.id, vals.data(), (int64_t)vals.size()))) return r;
        it->second.loaded = true;
        loaded++;
    }
    for (const auto& kv : slots)
        if (!kv.second.loaded) return fail_ctx(c, AARH_ERR_CHECKPOINT, "checkpoint lacks tensor " + kv.first);
    if (out_loaded) *out_loaded = loaded;
    return AARH_OK;
}

// IEEE binary16 nearest value, ties to even (the conversion of a float to _Float16).
uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // 65520 and above round to infinity
    if (ax < 0x38800000u) {                                    // below 2^-14: a multiple of 2^-24
        float a;
        memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint32_t)std::nearbyint(a * 16777216.0f));
    }
    const uint32_t m = ax + 0xFFFu + ((ax >> 13) & 1u) - (112u << 23);
    return (uint16_t)(sign | (m >> 13));
}

}  // namespace

extern "C" {

const char* aarh_host_last_error(void) { return g_host_err.c_str(); }

int aarh_load_gguf(aarh_ctx* c, const char* path, int32_t* out_loaded) {
    if (!c || !path) return AARH_ERR_CONFIG;
    Gguf g;
    std::string err;
    int r = gguf_open(path, g, err);
    if (r) return fail_ctx(c, r, err);
    if ((r = check_gguf_config(c, g.meta))) return r;
    return load_gguf_into(c, g, out_loaded);
}

int aarh_load_safetensors(aarh_ctx* c, const char* path, int32_t* out_loaded) {
    if (!c || !path) return AARH_ERR_CONFIG;
    return load_safetensors_into(c, path, out_loaded);
}

int aarh_lat_load_gguf(aarh_lat_ctx* c, const char* path, int32_t* out_loaded) {
    if (!c || !path) return AARH_ERR_CONFIG;
    Gguf g;
    std::string err;
    int r = gguf_open(path, g, err);
    if (r) return fail_ctx(c, r, err);
    if ((r = check_lat_gguf_config(c, g.meta))) return r;
    return load_gguf_into(c, g, out_loaded);
}

int aarh_lat_load_safetensors(aarh_lat_ctx* c, const char* path, int32_t* out_loaded) {
    if (!c || !path) return AARH_ERR_CONFIG;
    return load_safetensors_into(c, path, out_loaded);
}

int aarh_lat_gguf_config(const char* path, aarh_lat_config* out) {
    if (!path || !out) {
        g_host_err = "null path or config";
        return AARH_ERR_CONFIG;
    }
    Gguf g;
    std::string err;
    int r = gguf_open(path, g, err);
    if (r) return fail_ctx((aarh_ctx*)nullptr, r, err);
    if ((r = lat_config_from_json(g.meta, out, err))) return fail_ctx((aarh_ctx*)nullptr, r, err);
    return AARH_OK;
}

// PackedInt4Tensor (quant/src/types.rs:79-90) -> the device's INT4 g128 parameters.
// Checks follow dequantise_packed_i4_to_vec (int4.rs:70-91): a non-zero group size,
// ceil(numel / group_size) scales and zeros, and enough packed bytes for the shape.
// The device layout then needs the last dimension and the group size to be multiples
// of 128 (a reference group covers whole 128-column device groups), finite fp16 scales
// and integral zero points below 1024 in magnitude ((q - zero) stays exact in fp16).
int aarh_packed_i4_params(const int64_t* shape, int32_t ndims, int64_t group_size, int64_t data_len,
                          const float* scales, const float* zeros, int64_t n_groups, uint16_t* scales_f16,
                          uint16_t* zeros_f16) {
    char msg[256];
    auto bad = [&](int code) {
        g_host_err = msg;
        return code;
    };
    if (!shape || !scales || !zeros || !scales_f16 || !zeros_f16) {
        snprintf(msg, sizeof(msg), "null PackedInt4Tensor field");
        return bad(AARH_ERR_CONFIG);
    }
    if (ndims < 1 || ndims > 8) {
        snprintf(msg, sizeof(msg), "int4 tensor rank %d is not supported (1 to 8 dimensions)", ndims);
        return bad(AARH_ERR_SHAPE);
    }
    int64_t n = 1;
    for (int i = 0; i < ndims; i++) {
        if (shape[i] <= 0 || n > ((int64_t)1 << 40) / shape[i]) {
            snprintf(msg, sizeof(msg), "int4 tensor dimension %d has size %lld", i, (long long)shape[i]);
            return bad(AARH_ERR_SHAPE);
        }
        n *= shape[i];
    }
    if (group_size <= 0) {
        snprintf(msg, sizeof(msg), "group_size must be non-zero");
        return bad(AARH_ERR_CONFIG);
    }
    const int64_t expected = (n + group_size - 1) / group_size;
    if (n_groups != expected) {
        snprintf(msg, sizeof(msg), "expected %lld int4 groups, got %lld scales and %lld zeros", (long long)expected,
                 (long long)n_groups, (long long)n_groups);
        return bad(AARH_ERR_SHAPE);
    }
    if (data_len < 0 || data_len < (n + 1) / 2) {
        snprintf(msg, sizeof(msg), "int4 tensor holds %lld values but its shape has %lld elements",
                 (long long)(data_len < 0 ? 0 : 2 * data_len), (long long)n);
        return bad(AARH_ERR_SHAPE);
    }
    const int64_t cols = shape[ndims - 1], rows = n / cols;
    if (cols % 128) {
        snprintf(msg, sizeof(msg), "last dimension %lld is not a multiple of 128 (the device's INT4 group width)",
                 (long long)cols);
        return bad(AARH_ERR_UNSUPPORTED);
    }
    if (group_size % 128) {
        snprintf(msg, sizeof(msg),
                 "group_size %lld is not a multiple of 128: the device stores one scale and zero per 128 columns",
                 (long long)group_size);
        return bad(AARH_ERR_UNSUPPORTED);
    }
    for (int64_t g = 0; g < n_groups; g++) {
        const float sc = scales[g], z = zeros[g];
        const uint16_t h = f32_to_f16_rne(sc);
        if (!std::isfinite(sc) || (h & 0x7C00u) == 0x7C00u) {
            snprintf(msg, sizeof(msg), "scale %g of int4 group %lld has no finite fp16 value", (double)sc, (long long)g);
            return bad(AARH_ERR_UNSUPPORTED);
        }
        if (!(std::fabs(z) < 1024.0f) || z != std::nearbyint(z)) {
            snprintf(msg, sizeof(msg), "zero point %g of int4 group %lld is not an integer below 1024 in magnitude",
                     (double)z, (long long)g);
            return bad(AARH_ERR_UNSUPPORTED);
        }
    }
    const int64_t G = cols / 128;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t g = 0; g < G; g++) {
            const int64_t src = (r * cols + 128 * g) / group_size;
            scales_f16[r * G + g] = f32_to_f16_rne(scales[src]);
            zeros_f16[r * G + g] = f32_to_f16_rne(zeros[src]);
        }
    return AARH_OK;
}

int aarh_gguf_config(const char* path, aarh_model_config* out) {
    if (!path || !out) {
        g_host_err = "null path or config";
        return AARH_ERR_CONFIG;
    }
    Gguf g;
    std::string err;
    int r = gguf_open(path, g, err);
    if (r) return fail_ctx((aarh_ctx*)nullptr, r, err);
    const JVal* cfg = g.meta.get("config");
    if (!cfg || cfg->kind != JVal::OBJ) return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_CHECKPOINT, "GGUF metadata has no model config");
    const struct {
        const char* key;
        int32_t* dst;
    } ints[] = {{"vocab_size", &out->vocab_size}, {"hidden_dim", &out->hidden_dim}, {"ffn_dim", &out->ffn_dim},
                {"n_layers", &out->n_layers},     {"n_heads", &out->n_heads},       {"n_kv_heads", &out->n_kv_heads},
                {"max_seq_len", &out->max_seq_len}};
    for (const auto& fld : ints) {
        int64_t v = 0;
        if (!json_i64(cfg->get(fld.key), &v) || v < 0 || v > INT32_MAX)
            return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_CHECKPOINT, std::string("GGUF config lacks a valid ") + fld.key);
        *fld.dst = (int32_t)v;
    }
    const JVal* th = cfg->get("rope_theta");
    const JVal* ep = cfg->get("norm_eps");
    if (!th || th->kind != JVal::NUM || !ep || ep->kind != JVal::NUM)
        return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_CHECKPOINT, "GGUF config lacks rope_theta / norm_eps");
    out->rope_theta = (float)th->num;
    out->norm_eps = (float)ep->num;
    const JVal* tie = cfg->get("tie_embeddings");
    if (!tie || tie->kind != JVal::BOOL) return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_CHECKPOINT, "GGUF config lacks tie_embeddings");
    out->untied_lm_head = tie->b ? 0 : 1;
    out->num_future_tokens = 0;
    const JVal* mtp = cfg->get("mtp");
    if (mtp && mtp->kind == JVal::OBJ) {
        int64_t nft = 0;
        if (json_i64(mtp->get("num_future_tokens"), &nft) && nft > 0 && nft <= 64) out->num_future_tokens = (int32_t)nft;
    }
    return AARH_OK;
}

int aarh_gguf_rope_scaling(const char* path, aarh_rope_scaling* out) {
    if (!path || !out) {
        g_host_err = "null path or output";
        return AARH_ERR_CONFIG;
    }
    Gguf g;
    std::string err;
    int r = gguf_open(path, g, err);
    if (r) return fail_ctx((aarh_ctx*)nullptr, r, err);
    const JVal* cfg = g.meta.get("config");
    if (!cfg || cfg->kind != JVal::OBJ) return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_CHECKPOINT, "GGUF metadata has no model config");
    if ((r = parse_rope_scaling(cfg, out, err))) return fail_ctx((aarh_ctx*)nullptr, r, err);
    return AARH_OK;
}

int aarh_gguf_read_tensor(const char* path, const char* name, float* out, int64_t cap, int64_t* out_numel,
                          int32_t* out_ndims, int64_t* out_shape, int32_t* out_encoding) {
    if (!path || !name) {
        g_host_err = "null path or name";
        return AARH_ERR_CONFIG;
    }
    Gguf g;
    std::string err;
    int r = gguf_open(path, g, err);
    if (r) return fail_ctx((aarh_ctx*)nullptr, r, err);
    for (const GgufTensor& t : g.tensors) {
        if (t.name != name) continue;
        const int64_t n = numel(t.shape);
        if (out_numel) *out_numel = n;
        if (out_ndims) *out_ndims = (int32_t)t.shape.size();
        if (out_shape)
            for (size_t d = 0; d < t.shape.size(); d++) out_shape[d] = t.shape[d];
        if (out_encoding) *out_encoding = t.enc;
        if (!out) return AARH_OK;
        if (cap < n) return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_SHAPE, "output buffer too small for " + t.name);
        std::vector<float> vals;
        if ((r = gguf_decode(g, t, vals, err))) return fail_ctx((aarh_ctx*)nullptr, r, err);
        memcpy(out, vals.data(), (size_t)n * 4);
        return AARH_OK;
    }
    return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_SHAPE, std::string("no tensor ") + name + " in " + path);
}

int aarh_safetensors_read_tensor(const char* path, const char* name, float* out, int64_t cap, int64_t* out_numel,
                                 int32_t* out_ndims, int64_t* out_shape) {
    if (!path || !name) {
        g_host_err = "null path or name";
        return AARH_ERR_CONFIG;
    }
    File file;
    std::vector<StTensor> ts;
    uint64_t data_off = 0;
    std::string err;
    int r = st_open(path, file, ts, &data_off, err);
    if (r) return fail_ctx((aarh_ctx*)nullptr, r, err);
    for (const StTensor& t : ts) {
        if (t.name != name) continue;
        if (t.shape.size() > 8) return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_SHAPE, "tensor " + t.name + " has more than 8 dims");
        const int64_t n = numel(t.shape);
        if (out_numel) *out_numel = n;
        if (out_ndims) *out_ndims = (int32_t)t.shape.size();
        if (out_shape)
            for (size_t d = 0; d < t.shape.size(); d++) out_shape[d] = t.shape[d];
        if (!out) return AARH_OK;
        if (cap < n) return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_SHAPE, "output buffer too small for " + t.name);
        std::vector<float> vals;
        if ((r = st_decode(file, data_off, t, vals, err))) return fail_ctx((aarh_ctx*)nullptr, r, err);
        memcpy(out, vals.data(), (size_t)n * 4);
        return AARH_OK;
    }
    return fail_ctx((aarh_ctx*)nullptr, AARH_ERR_SHAPE, std::string("no tensor ") + name + " in " + path);
}

}  // extern "C"
