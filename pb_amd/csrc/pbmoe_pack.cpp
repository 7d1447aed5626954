// Expert pack metadata reader: layer_NN.json, the serde_json form of
// ExpertLayerPackMetadata (experts/mod.rs:283-454), read and validated as
// read_expert_layer_pack_metadata + ExpertLayerPackMetadata::validate do
// (experts/mod.rs:2501-2519, 372-429).  The JSON reader is a small
// recursive-descent parser for exactly what serde_json writes (objects,
// arrays, strings with escapes, integers, floats, booleans, null); unknown
// fields are ignored, as serde does by default.
#include "pbmoe_pack.h"

#include <errno.h>
#include <sys/stat.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>

#include "../../include/pbmoe.h"

namespace pbmoe {
namespace pack {

const char* const FORMAT_PBQ4_V1 = "PBQ4EXPERT_LAYER_V1";
const char* const FORMAT_PBQ4_V2 = "PBQ4EXPERT_LAYER_V2";
const char* const FORMAT_FIXED_Q4 = "FIXED_Q4_EXPERT_LAYER_V1";
const char* const FORMAT_FIXED_MXFP4 = "FIXED_MXFP4_EXPERT_LAYER_V1";
const char* const FORMAT_FIXED_DENSE = "FIXED_DENSE_EXPERT_LAYER_V1";
const char* const FORMAT_FIXED_DEEPSEEK_GGUF = "FIXED_DEEPSEEK_GGUF_EXPERT_LAYER_V1";

namespace {

struct Json {
    enum Kind { Null, Bool, Int, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    uint64_t u = 0; // Int: non-negative integer without fraction or exponent
    bool neg = false;
    double num = 0.0;
    std::string s;
    std::vector<Json> a;
    std::vector<std::pair<std::string, Json>> o;

    const Json* get(const char* key) const
    {
        for (const auto& kv : o)
            if (kv.first == key)
                return &kv.second;
        return nullptr;
    }
};

class Parser {
public:
    Parser(const char* p, const char* end) : p_(p), end_(end) {}

    bool parse(Json* out, std::string* err)
    {
        if (!value(out, 0) || (skip(), p_ != end_)) {
            if (err_.empty())
                err_ = "trailing characters";
            *err = err_ + " at byte " + std::to_string(offset());
            return false;
        }
        return true;
    }

private:
    const char* p_;
    const char* end_;
    const char* start_ = p_; // declared after p_: initialised from it
    std::string err_;

    size_t offset() const { return (size_t)(p_ - start_); }

    void skip()
    {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r'))
            ++p_;
    }

    bool fail(const char* what)
    {
        if (err_.empty())
            err_ = what;
        return false;
    }

    bool literal(const char* word)
    {
        const size_t n = strlen(word);
        if ((size_t)(end_ - p_) < n || memcmp(p_, word, n) != 0)
            return fail("invalid literal");
        p_ += n;
        return true;
    }

    static void put_utf8(std::string& s, uint32_t cp)
    {
        if (cp < 0x80) {
            s.push_back((char)cp);
        } else if (cp < 0x800) {
            s.push_back((char)(0xC0 | (cp >> 6)));
            s.push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            s.push_back((char)(0xE0 | (cp >> 12)));
            s.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s.push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            s.push_back((char)(0xF0 | (cp >> 18)));
            s.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            s.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            s.push_back((char)(0x80 | (cp & 0x3F)));
        }
    }

    bool hex4(uint32_t* v)
    {
        if (end_ - p_ < 4)
            return fail("truncated \\u escape");
        uint32_t r = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            r <<= 4;
            if (c >= '0' && c <= '9')
                r |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f')
                r |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F')
                r |= (uint32_t)(c - 'A' + 10);
            else
                return fail("invalid \\u escape");
        }
        *v = r;
        return true;
    }

    bool string(std::string* s)
    {
        if (p_ >= end_ || *p_ != '"')
            return fail("expected string");
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            const unsigned char c = (unsigned char)*p_;
            if (c < 0x20)
                return fail("control character in string");
            if (c != '\\') {
                s->push_back((char)c);
                ++p_;
                continue;
            }
            if (++p_ >= end_)
                return fail("truncated escape");
            const char e = *p_++;
            switch (e) {
            case '"': s->push_back('"'); break;
            case '\\': s->push_back('\\'); break;
            case '/': s->push_back('/'); break;
            case 'b': s->push_back('\b'); break;
            case 'f': s->push_back('\f'); break;
            case 'n': s->push_back('\n'); break;
            case 'r': s->push_back('\r'); break;
            case 't': s->push_back('\t'); break;
            case 'u': {
                uint32_t cp;
                if (!hex4(&cp))
                    return false;
                if (cp >= 0xD800 && cp < 0xDC00) { // surrogate pair
                    uint32_t lo;
                    if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u')
                        return fail("unpaired surrogate");
                    p_ += 2;
                    if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000)
                        return fail("invalid surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    return fail("unpaired surrogate");
                }
                put_utf8(*s, cp);
                break;
            }
            default: return fail("invalid escape");
            }
        }
        if (p_ >= end_)
            return fail("unterminated string");
        ++p_;
        return true;
    }

    bool number(Json* v)
    {
        const char* b = p_;
        bool neg = false, frac = false;
        if (p_ < end_ && *p_ == '-')
            neg = true, ++p_;
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9'))
            return fail("invalid number");
        if (*p_ == '0' && p_ + 1 < end_ && p_[1] >= '0' && p_[1] <= '9')
            return fail("leading zero");
        uint64_t u = 0;
        bool overflow = false;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_ - '0');
            if (u > (UINT64_MAX - d) / 10)
                overflow = true;
            u = u * 10 + d;
            ++p_;
        }
        if (p_ < end_ && *p_ == '.') {
            frac = true, ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9'))
                return fail("invalid fraction");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9')
                ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true, ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-'))
                ++p_;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9'))
                return fail("invalid exponent");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9')
                ++p_;
        }
        v->num = strtod(std::string(b, p_).c_str(), nullptr);
        v->neg = neg;
        if (!frac && !overflow) {
            v->kind = Json::Int;
            v->u = u;
        } else {
            v->kind = Json::Num;
        }
        return true;
    }

    bool value(Json* v, int depth)
    {
        if (depth > 64)
            return fail("nesting too deep");
        skip();
        if (p_ >= end_)
            return fail("unexpected end of input");
        switch (*p_) {
        case '{': {
            ++p_;
            v->kind = Json::Obj;
            skip();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                skip();
                std::pair<std::string, Json> kv;
                if (!string(&kv.first))
                    return false;
                skip();
                if (p_ >= end_ || *p_ != ':')
                    return fail("expected ':'");
                ++p_;
                if (!value(&kv.second, depth + 1))
                    return false;
                v->o.push_back(std::move(kv));
                skip();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        case '[': {
            ++p_;
            v->kind = Json::Arr;
            skip();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                Json e;
                if (!value(&e, depth + 1))
                    return false;
                v->a.push_back(std::move(e));
                skip();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        case '"':
            v->kind = Json::Str;
            return string(&v->s);
        case 't':
            v->kind = Json::Bool, v->b = true;
            return literal("true");
        case 'f':
            v->kind = Json::Bool, v->b = false;
            return literal("false");
        case 'n':
            v->kind = Json::Null;
            return literal("null");
        default:
            return number(v);
        }
    }
};

// Field readers with serde's required/default semantics.
struct Fields {
    const Json& obj;
    const char* what;
    std::string* err;

    bool u64(const char* key, uint64_t* out, bool required = true)
    {
        const Json* v = obj.get(key);
        if (!v) {
            if (required)
                *err = std::string(what) + ": missing field `" + key + "`";
            return !required;
        }
        if (v->kind != Json::Int || v->neg) {
            *err = std::string(what) + ": field `" + key + "` is not a non-negative integer";
            return false;
        }
        *out = v->u;
        return true;
    }

    bool str(const char* key, std::string* out, bool required = true)
    {
        const Json* v = obj.get(key);
        if (!v) {
            if (required)
                *err = std::string(what) + ": missing field `" + key + "`";
            return !required;
        }
        if (v->kind != Json::Str) {
            *err = std::string(what) + ": field `" + key + "` is not a string";
            return false;
        }
        *out = v->s;
        return true;
    }

    const Json* arr(const char* key)
    {
        const Json* v = obj.get(key);
        if (!v) {
            *err = std::string(what) + ": missing field `" + key + "`";
            return nullptr;
        }
        if (v->kind != Json::Arr) {
            *err = std::string(what) + ": field `" + key + "` is not an array";
            return nullptr;
        }
        return v;
    }
};

bool to_record(const Json& j, Record* r, std::string* err)
{
    if (j.kind != Json::Obj) {
        *err = "record is not an object";
        return false;
    }
    Fields f{j, "record", err};
    if (!f.str("tensor", &r->tensor) || !f.str("dtype", &r->dtype))
        return false;
    const Json* shape = f.arr("shape");
    if (!shape)
        return false;
    for (const Json& d : shape->a) {
        if (d.kind != Json::Int || d.neg) {
            *err = "record " + r->tensor + ": shape entry is not a non-negative integer";
            return false;
        }
        r->shape.push_back(d.u);
    }
    const Json* so = f.arr("source_offsets");
    if (!so)
        return false;
    if (so->a.size() != 2) {
        *err = "record " + r->tensor + ": source_offsets must hold two integers";
        return false;
    }
    for (const Json& d : so->a)
        if (d.kind != Json::Int || d.neg) {
            *err = "record " + r->tensor + ": source_offsets entry is not a non-negative integer";
            return false;
        }
    if (const Json* h = j.get("source_hash"))
        if (h->kind != Json::Str && h->kind != Json::Null) {
            *err = "record " + r->tensor + ": source_hash is not a string";
            return false;
        }
    r->scale_bias_dtype = "F32";
    return f.u64("record_offset", &r->record_offset) && f.u64("packed_bytes", &r->packed_bytes) &&
           f.u64("groups", &r->groups) && f.u64("group_size", &r->group_size) &&
           f.str("scale_bias_dtype", &r->scale_bias_dtype, false);
}

bool to_pack(const Json& j, Pack* p, std::string* err)
{
    if (j.kind != Json::Obj) {
        *err = "pack is not an object";
        return false;
    }
    Fields f{j, "pack", err};
    if (!f.u64("layer", &p->layer) || !f.u64("expert", &p->expert) ||
        !f.u64("packed_bytes", &p->packed_bytes, false))
        return false;
    const Json* recs = f.arr("records");
    if (!recs)
        return false;
    for (const Json& r : recs->a) {
        Record rec;
        if (!to_record(r, &rec, err))
            return false;
        p->records.push_back(std::move(rec));
    }
    return true;
}

bool known_format(const std::string& f)
{
    for (const char* k : {FORMAT_PBQ4_V1, FORMAT_PBQ4_V2, FORMAT_FIXED_Q4, FORMAT_FIXED_MXFP4,
                          FORMAT_FIXED_DENSE, FORMAT_FIXED_DEEPSEEK_GGUF})
        if (f == k)
            return true;
    return false;
}

} // namespace

const Pack* LayerMeta::pack_for(uint64_t expert) const
{
    for (const Pack& p : packs)
        if (p.expert == expert)
            return &p;
    return nullptr;
}

std::string layer_bin_path(const std::string& root, uint32_t layer)
{
    char name[32];
    snprintf(name, sizeof(name), "layer_%02u.bin", layer);
    return root + "/" + name;
}

std::string layer_json_path(const std::string& root, uint32_t layer)
{
    char name[32];
    snprintf(name, sizeof(name), "layer_%02u.json", layer);
    return root + "/" + name;
}

int64_t file_size(const std::string& path)
{
    struct stat st;
    if (stat(path.c_str(), &st) != 0)
        return -1;
    if (!S_ISREG(st.st_mode)) {
        errno = EINVAL;
        return -1;
    }
    return (int64_t)st.st_size;
}

int read_layer_meta(const std::string& root, uint32_t layer, LayerMeta* out, std::string* err)
{
    const std::string path = layer_json_path(root, layer);
    FILE* fp = fopen(path.c_str(), "rb");
    if (!fp) {
        *err = "expert metadata " + path + " is missing: " + strerror(errno);
        return PBMOE_ERR_IO;
    }
    std::string text;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), fp)) > 0) {
        text.append(buf, n);
        if (text.size() > (256u << 20)) {
            fclose(fp);
            *err = "expert metadata " + path + " exceeds 256 MiB";
            return PBMOE_ERR_FORMAT;
        }
    }
    const bool read_err = ferror(fp) != 0;
    fclose(fp);
    if (read_err) {
        *err = "failed to read expert metadata " + path;
        return PBMOE_ERR_IO;
    }
    Json root_v;
    std::string perr;
    if (!Parser(text.data(), text.data() + text.size()).parse(&root_v, &perr)) {
        *err = "failed to parse expert metadata " + path + ": " + perr;
        return PBMOE_ERR_FORMAT;
    }
    if (root_v.kind != Json::Obj) {
        *err = "failed to parse expert metadata " + path + ": not an object";
        return PBMOE_ERR_FORMAT;
    }
    LayerMeta m;
    std::string ferr;
    Fields f{root_v, "layer metadata", &ferr};
    const Json* packs = nullptr;
    if (!f.str("format", &m.format) || !f.u64("layer", &m.layer) || !f.u64("expert_size", &m.expert_size) ||
        !f.u64("experts", &m.experts) || !(packs = f.arr("packs"))) {
        *err = "failed to parse expert metadata " + path + ": " + ferr;
        return PBMOE_ERR_FORMAT;
    }
    for (const Json& pj : packs->a) {
        Pack p;
        if (!to_pack(pj, &p, &ferr)) {
            *err = "failed to parse expert metadata " + path + ": " + ferr;
            return PBMOE_ERR_FORMAT;
        }
        m.packs.push_back(std::move(p));
    }
    // ExpertLayerPackMetadata::validate (experts/mod.rs:372-429)
    if (!known_format(m.format)) {
        *err = "expert metadata " + path + " has unsupported format " + m.format;
        return PBMOE_ERR_FORMAT;
    }
    if (m.layer != layer) {
        *err = "expert metadata " + path + " describes layer " + std::to_string(m.layer) +
               ", expected layer " + std::to_string(layer);
        return PBMOE_ERR_FORMAT;
    }
    if (m.expert_size == 0) {
        *err = "expert metadata " + path + " has zero expert_size";
        return PBMOE_ERR_FORMAT;
    }
    if (m.experts == 0) {
        *err = "expert metadata " + path + " has zero experts";
        return PBMOE_ERR_FORMAT;
    }
    std::set<uint64_t> seen;
    for (const Pack& p : m.packs) {
        if (p.layer != layer) { // validate_expert_pack_metadata (experts/mod.rs:2460-2476)
            *err = "expert metadata " + path + " describes layer " + std::to_string(p.layer) + " expert " +
                   std::to_string(p.expert) + ", expected layer " + std::to_string(layer) + " expert " +
                   std::to_string(p.expert);
            return PBMOE_ERR_FORMAT;
        }
        if (p.expert >= m.experts) {
            *err = "expert metadata " + path + " describes expert " + std::to_string(p.expert) +
                   " outside 0.." + std::to_string(m.experts);
            return PBMOE_ERR_FORMAT;
        }
        if (!seen.insert(p.expert).second) {
            *err = "expert metadata " + path + " has duplicate expert " + std::to_string(p.expert);
            return PBMOE_ERR_FORMAT;
        }
        if (p.packed_bytes > m.expert_size) {
            *err = "expert metadata " + path + " expert " + std::to_string(p.expert) + " length " +
                   std::to_string(p.packed_bytes) + " exceeds slot size " + std::to_string(m.expert_size);
            return PBMOE_ERR_FORMAT;
        }
    }
    *out = std::move(m);
    return 0;
}

} // namespace pack
} // namespace pbmoe
