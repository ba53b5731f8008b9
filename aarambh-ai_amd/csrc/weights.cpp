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

std::map<std::string, Slot> context_slots(aarh_ctx* ctx) {
    std::map<std::string, Slot> m;
    char name[256];
    const int n = aarh_num_tensors(ctx);
    for (int id = 0; id < n; id++) {
        int64_t r = 0, c = 0;
        int32_t kind = 0;
        if (aarh_tensor_info(ctx, id, name, sizeof(name), &r, &c, &kind) == AARH_OK) m[name] = Slot{id, r, c};
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

// Set by the library's runtime (runtime.cpp): the context's error text.
namespace aarh {
int ctx_fail(aarh_ctx* c, int code, const char* msg);
}

namespace {

int fail_ctx(aarh_ctx* c, int code, const std::string& msg) {
    if (c) return aarh::ctx_fail(c, code, msg.c_str());
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
    auto slots = context_slots(c);
    int loaded = 0;
    std::vector<float> vals;
    for (const GgufTensor& t : g.tensors) {
        auto it = slots.find(t.name);
        if (it == slots.end()) continue;  // tensors of other layer kinds (VarBuilder reads by name)
        if (!shape_matches(t.shape, it->second))
            return fail_ctx(c, AARH_ERR_SHAPE, "checkpoint tensor " + t.name + " has a shape the model does not expect");
        if ((r = gguf_decode(g, t, vals, err))) return fail_ctx(c, r, err);
        if ((r = aarh_load_tensor_f32(c, it->second.id, vals.data(), (int64_t)vals.size()))) return r;
        it->second.loaded = true;
        loaded++;
    }
    for (const auto& kv : slots)
        if (!kv.second.loaded) return fail_ctx(c, AARH_ERR_CHECKPOINT, "checkpoint lacks tensor " + kv.first);
    if (out_loaded) *out_loaded = loaded;
    return AARH_OK;
}

int aarh_load_safetensors(aarh_ctx* c, const char* path, int32_t* out_loaded) {
    if (!c || !path) return AARH_ERR_CONFIG;
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
        if ((r = aarh_load_tensor_f32(c, it->second.id, vals.data(), (int64_t)vals.size()))) return r;
        it->second.loaded = true;
        loaded++;
    }
    for (const auto& kv : slots)
        if (!kv.second.loaded) return fail_ctx(c, AARH_ERR_CHECKPOINT, "checkpoint lacks tensor " + kv.first);
    if (out_loaded) *out_loaded = loaded;
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
    if (r) return fail_ctx(nullptr, r, err);
    const JVal* cfg = g.meta.get("config");
    if (!cfg || cfg->kind != JVal::OBJ) return fail_ctx(nullptr, AARH_ERR_CHECKPOINT, "GGUF metadata has no model config");
    const struct {
        const char* key;
        int32_t* dst;
    } ints[] = {{"vocab_size", &out->vocab_size}, {"hidden_dim", &out->hidden_dim}, {"ffn_dim", &out->ffn_dim},
                {"n_layers", &out->n_layers},     {"n_heads", &out->n_heads},       {"n_kv_heads", &out->n_kv_heads},
                {"max_seq_len", &out->max_seq_len}};
    for (const auto& fld : ints) {
        int64_t v = 0;
        if (!json_i64(cfg->get(fld.key), &v) || v < 0 || v > INT32_MAX)
            return fail_ctx(nullptr, AARH_ERR_CHECKPOINT, std::string("GGUF config lacks a valid ") + fld.key);
        *fld.dst = (int32_t)v;
    }
    const JVal* th = cfg->get("rope_theta");
    const JVal* ep = cfg->get("norm_eps");
    if (!th || th->kind != JVal::NUM || !ep || ep->kind != JVal::NUM)
        return fail_ctx(nullptr, AARH_ERR_CHECKPOINT, "GGUF config lacks rope_theta / norm_eps");
    out->rope_theta = (float)th->num;
    out->norm_eps = (float)ep->num;
    const JVal* tie = cfg->get("tie_embeddings");
    if (!tie || tie->kind != JVal::BOOL) return fail_ctx(nullptr, AARH_ERR_CHECKPOINT, "GGUF config lacks tie_embeddings");
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
    if (r) return fail_ctx(nullptr, r, err);
    const JVal* cfg = g.meta.get("config");
    if (!cfg || cfg->kind != JVal::OBJ) return fail_ctx(nullptr, AARH_ERR_CHECKPOINT, "GGUF metadata has no model config");
    if ((r = parse_rope_scaling(cfg, out, err))) return fail_ctx(nullptr, r, err);
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
    if (r) return fail_ctx(nullptr, r, err);
    for (const GgufTensor& t : g.tensors) {
        if (t.name != name) continue;
        const int64_t n = numel(t.shape);
        if (out_numel) *out_numel = n;
        if (out_ndims) *out_ndims = (int32_t)t.shape.size();
        if (out_shape)
            for (size_t d = 0; d < t.shape.size(); d++) out_shape[d] = t.shape[d];
        if (out_encoding) *out_encoding = t.enc;
        if (!out) return AARH_OK;
        if (cap < n) return fail_ctx(nullptr, AARH_ERR_SHAPE, "output buffer too small for " + t.name);
        std::vector<float> vals;
        if ((r = gguf_decode(g, t, vals, err))) return fail_ctx(nullptr, r, err);
        memcpy(out, vals.data(), (size_t)n * 4);
        return AARH_OK;
    }
    return fail_ctx(nullptr, AARH_ERR_SHAPE, std::string("no tensor ") + name + " in " + path);
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
    if (r) return fail_ctx(nullptr, r, err);
    for (const StTensor& t : ts) {
        if (t.name != name) continue;
        if (t.shape.size() > 8) return fail_ctx(nullptr, AARH_ERR_SHAPE, "tensor " + t.name + " has more than 8 dims");
        const int64_t n = numel(t.shape);
        if (out_numel) *out_numel = n;
        if (out_ndims) *out_ndims = (int32_t)t.shape.size();
        if (out_shape)
            for (size_t d = 0; d < t.shape.size(); d++) out_shape[d] = t.shape[d];
        if (!out) return AARH_OK;
        if (cap < n) return fail_ctx(nullptr, AARH_ERR_SHAPE, "output buffer too small for " + t.name);
        std::vector<float> vals;
        if ((r = st_decode(file, data_off, t, vals, err))) return fail_ctx(nullptr, r, err);
        memcpy(out, vals.data(), (size_t)n * 4);
        return AARH_OK;
    }
    return fail_ctx(nullptr, AARH_ERR_SHAPE, std::string("no tensor ") + name + " in " + path);
}

}  // extern "C"
