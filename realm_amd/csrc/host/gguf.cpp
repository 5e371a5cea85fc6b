// GGUF model images on the host side of the boundary: the header, the
// metadata key/values and the tensor table parsed as the reference parses them
// (crates/realm-core/src/formats/gguf.rs:111-160, 300-480), the reference's
// transformer-config extraction (gguf.rs:212-280), and the image's 2-D Q4_K /
// Q6_K / Q8_0 tensors registered once as resident device weights, keyed by
// tensor name, in place of ModelStorage's per-call tensor copies
// (crates/realm-runtime/src/model_storage.rs:386-487).
//
// Parsing touches no device.  Where this module differs from the reference it
// follows the GGUF format the reference reads:
//  * tensor bytes start at the data section, the end of the tensor table
//    rounded up to general.alignment (32 when the key is absent, the
//    reference's fixed value, gguf.rs:165-175), plus the tensor's offset
//    (as TensorLoader, tensor_loader.rs:76; ModelStorage::store_model reads
//    at the bare offset);
//  * a Q8_0 tensor holds 34-byte blocks (BlockQ8_0, quant.rs:52-59), where
//    TensorDesc::new counts 33 (tensor.rs:145-150), and Q4_0 / Q4_1 tensors
//    18- and 20-byte blocks (quant.rs:10-28), where it counts 16.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "realm_hip.h"

// realm_hip.cpp: sets the calling thread's last-error message, returns code
int realm_set_error(int code, const std::string &msg);
// Free device memory of the library's device, in bytes (initialises it).
int realm_device_free_bytes(size_t *bytes);

namespace {

enum : uint32_t {
    GGUF_MAGIC = 0x46554747u, // "GGUF"
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};

// One metadata value: integers keep their bit pattern sign-extended or
// zero-extended into i64 (as_u32 truncates it, gguf.rs:50-62); arrays keep
// their element type and length.
struct MetaValue {
    uint32_t type = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    uint32_t elem_type = 0;
    uint64_t len = 0;
};

struct Tensor {
    std::string name;
    int32_t type = 0;
    std::vector<uint64_t> dims;
    uint64_t offset = 0;   // relative to the data section, as stored
    uint64_t abs = 0;      // data section + offset
    uint64_t nbytes = 0;   // 0 for types this module does not size
    uint64_t weight = 0;   // registered device weight (0: none)
};

struct Model {
    uint32_t version = 0;
    uint64_t tensor_count = 0, kv_count = 0, alignment = 32, data_offset = 0;
    std::unordered_map<std::string, MetaValue> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name; // last tensor of a name wins
};

std::mutex g_gguf_mu;
std::unordered_map<uint64_t, Model> g_models;
uint64_t g_next_model = 1;

// Little-endian reader over the image; every read is bounds-checked, and a
// read past the end is the reference's read_exact failure (Error::Io).
struct Reader {
    const uint8_t *p;
    size_t len, pos = 0;
    template <class T>
    int get(T *v)
    {
        if (len - pos < sizeof(T))
            return realm_set_error(REALM_IO_ERROR, "GGUF image ends inside the header");
        std::memcpy(v, p + pos, sizeof(T));
        pos += sizeof(T);
        return REALM_OK;
    }
    int str(std::string *s)
    {
        uint64_t n = 0;
        if (int rc = get(&n))
            return rc;
        if (n > len - pos)
            return realm_set_error(REALM_IO_ERROR, "GGUF image ends inside a string");
        s->assign(reinterpret_cast<const char *>(p + pos), (size_t)n);
        pos += (size_t)n;
        // String::from_utf8 (gguf.rs:300-305): invalid UTF-8 is a ParseError
        const unsigned char *c = reinterpret_cast<const unsigned char *>(s->data());
        for (size_t i = 0; i < s->size();) {
            const unsigned b = c[i];
            size_t k = b < 0x80 ? 1 : (b >> 5) == 6 ? 2 : (b >> 4) == 14 ? 3 : (b >> 3) == 30 ? 4 : 0;
            if (k == 0 || i + k > s->size())
                return realm_set_error(REALM_MODEL_PARSE_ERROR, "Invalid UTF-8 in GGUF string");
            uint32_t cp = k == 1 ? b : (b & (0x7Fu >> k));
            for (size_t j = 1; j < k; ++j) {
                if ((c[i + j] & 0xC0) != 0x80)
                    return realm_set_error(REALM_MODEL_PARSE_ERROR, "Invalid UTF-8 in GGUF string");
                cp = (cp << 6) | (c[i + j] & 0x3F);
            }
            const uint32_t min_cp[5] = {0, 0, 0x80, 0x800, 0x10000};
            if (cp < min_cp[k] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
                return realm_set_error(REALM_MODEL_PARSE_ERROR, "Invalid UTF-8 in GGUF string");
            i += k;
        }
        return REALM_OK;
    }
};

#define GG_TRY(x)                                                                                \
    do {                                                                                         \
        if (int rc_ = (x))                                                                       \
            return rc_;                                                                          \
    } while (0)

// A scalar of type t (gguf.rs:368-425; an array element may not itself be
// an array, as read_typed_value has no arm for it).
int read_scalar(Reader &r, uint32_t t, MetaValue *v)
{
    v->type = t;
    switch (t) {
    case V_U8: { uint8_t x = 0; GG_TRY(r.get(&x)); v->i = x; return REALM_OK; }
    case V_I8: { int8_t x = 0; GG_TRY(r.get(&x)); v->i = x; return REALM_OK; }
    case V_U16: { uint16_t x = 0; GG_TRY(r.get(&x)); v->i = x; return REALM_OK; }
    case V_I16: { int16_t x = 0; GG_TRY(r.get(&x)); v->i = x; return REALM_OK; }
    case V_U32: { uint32_t x = 0; GG_TRY(r.get(&x)); v->i = x; return REALM_OK; }
    case V_I32: { int32_t x = 0; GG_TRY(r.get(&x)); v->i = x; return REALM_OK; }
    case V_F32: { float x = 0; GG_TRY(r.get(&x)); v->f = x; return REALM_OK; }
    case V_BOOL: { uint8_t x = 0; GG_TRY(r.get(&x)); v->i = x != 0; return REALM_OK; }
    case V_STR: return r.str(&v->s);
    case V_U64: { uint64_t x = 0; GG_TRY(r.get(&x)); v->i = (int64_t)x; return REALM_OK; }
    case V_I64: { int64_t x = 0; GG_TRY(r.get(&x)); v->i = x; return REALM_OK; }
    case V_F64: { double x = 0; GG_TRY(r.get(&x)); v->f = x; return REALM_OK; }
    default:
        return realm_set_error(REALM_MODEL_PARSE_ERROR,
                               "Unknown metadata value type: " + std::to_string(t));
    }
}

int read_value(Reader &r, MetaValue *v)
{
    uint32_t t = 0;
    GG_TRY(r.get(&t));
    if (t != V_ARR)
        return read_scalar(r, t, v);
    v->type = V_ARR;
    GG_TRY(r.get(&v->elem_type));
    GG_TRY(r.get(&v->len));
    MetaValue e;
    for (uint64_t k = 0; k < v->len; ++k) {
        if (v->elem_type == V_ARR)
            return realm_set_error(REALM_MODEL_PARSE_ERROR, "Unknown typed value: 9");
        GG_TRY(read_scalar(r, v->elem_type, &e));
    }
    return REALM_OK;
}

// Bytes of a tensor of ggml type t with nel elements, for the types whose
// size this path relies on (tensor.rs:135-175, with the block sizes of
// quant.rs:10-70); 0 for the others, which are listed but never registered.
uint64_t tensor_bytes(int32_t t, uint64_t nel)
{
    switch (t) {
    case 0: return nel * 4;          // F32
    case 1: return nel * 2;          // F16
    case 2: return nel / 32 * 18;    // Q4_0 (BlockQ4_0; TensorDesc counts 16)
    case 3: return nel / 32 * 20;    // Q4_1 (BlockQ4_1; TensorDesc counts 16)
    case 6: return nel / 32 * 22;    // Q5_0
    case 7: return nel / 32 * 24;    // Q5_1
    case 8: return nel / 32 * 34;    // Q8_0
    case 9: return nel / 32 * 36;    // Q8_1
    case 12: return nel / 256 * 144; // Q4_K
    case 14: return nel / 256 * 210; // Q6_K
    default: return 0;
    }
}

int parse(const uint8_t *bytes, size_t len, Model *m)
{
    Reader r{bytes, len};
    uint32_t magic = 0;
    GG_TRY(r.get(&magic));
    if (magic != GGUF_MAGIC) {
        char buf[64];
        std::snprintf(buf, sizeof buf, "Invalid GGUF magic: 0x%08X", magic);
        return realm_set_error(REALM_MODEL_PARSE_ERROR, buf);
    }
    GG_TRY(r.get(&m->version));
    if (m->version < 2 || m->version > 3)
        return realm_set_error(REALM_MODEL_PARSE_ERROR,
                               "Unsupported GGUF version: " + std::to_string(m->version));
    GG_TRY(r.get(&m->tensor_count));
    GG_TRY(r.get(&m->kv_count));
    for (uint64_t i = 0; i < m->kv_count; ++i) {
        std::string key;
        GG_TRY(r.str(&key));
        MetaValue v;
        GG_TRY(read_value(r, &v));
        m->meta[key] = std::move(v); // a repeated key: the last value wins (HashMap insert)
    }
    for (uint64_t i = 0; i < m->tensor_count; ++i) {
        Tensor t;
        GG_TRY(r.str(&t.name));
        uint32_t nd = 0;
        GG_TRY(r.get(&nd));
        if (nd > (r.len - r.pos) / 8)
            return realm_set_error(REALM_IO_ERROR, "GGUF image ends inside a tensor shape");
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; ++d)
            GG_TRY(r.get(&t.dims[d]));
        uint32_t ty = 0;
        GG_TRY(r.get(&ty));
        t.type = (int32_t)ty;
        GG_TRY(r.get(&t.offset));
        // Shape::validate (tensor.rs:102-110)
        if (t.dims.empty())
            return realm_set_error(REALM_INVALID_ARGUMENT, "Invalid tensor shape: Shape cannot be empty");
        uint64_t nel = 1;
        for (uint64_t d : t.dims) {
            if (d == 0)
                return realm_set_error(REALM_INVALID_ARGUMENT,
                                       "Invalid tensor shape: Shape dimensions must be > 0");
            if (nel > UINT64_MAX / d)
                return realm_set_error(REALM_INVALID_ARGUMENT, "tensor " + t.name + " too large");
            nel *= d;
        }
        t.nbytes = tensor_bytes(t.type, nel);
        m->tensors.push_back(std::move(t));
    }
    auto al = m->meta.find("general.alignment");
    if (al != m->meta.end() && al->second.type == V_U32) {
        const uint64_t a = (uint64_t)al->second.i;
        if (a == 0 || (a & (a - 1)))
            return realm_set_error(REALM_MODEL_PARSE_ERROR,
                                   "general.alignment " + std::to_string(a) + " is not a power of two");
        m->alignment = a;
    }
    m->data_offset = (r.pos + m->alignment - 1) / m->alignment * m->alignment;
    for (size_t i = 0; i < m->tensors.size(); ++i) {
        Tensor &t = m->tensors[i];
        t.abs = m->data_offset + t.offset;
        m->by_name[t.name] = i;
    }
    return REALM_OK;
}

int get_model(uint64_t h, Model **out)
{
    auto it = g_models.find(h);
    if (it == g_models.end())
        return realm_set_error(REALM_INVALID_ARGUMENT, "unknown GGUF model handle " + std::to_string(h));
    *out = &it->second;
    return REALM_OK;
}

const MetaValue *meta_of(const Model &m, const std::string &key)
{
    auto it = m.meta.find(key);
    return it == m.meta.end() ? nullptr : &it->second;
}

bool is_int(uint32_t t)
{
    return t == V_U8 || t == V_I8 || t == V_U16 || t == V_I16 || t == V_U32 || t == V_I32 ||
           t == V_U64 || t == V_I64;
}

// MetadataValue::as_u32 / as_f32 / as_string (gguf.rs:50-85)
bool as_u32(const MetaValue *v, uint32_t *out)
{
    if (!v || !is_int(v->type))
        return false;
    *out = (uint32_t)(uint64_t)v->i;
    return true;
}
bool as_f32(const MetaValue *v, float *out)
{
    if (!v || (v->type != V_F32 && v->type != V_F64))
        return false;
    *out = (float)v->f;
    return true;
}

// The first key that holds a value of the wanted kind, else the default
// (the or_else chains of extract_config, gguf.rs:212-280).
uint32_t cfg_u32(const Model &m, const std::string &k1, const std::string &k2, uint32_t def)
{
    uint32_t v;
    const MetaValue *a = meta_of(m, k1);
    if (a)
        return as_u32(a, &v) ? v : def;
    return as_u32(meta_of(m, k2), &v) ? v : def;
}
float cfg_f32(const Model &m, const std::string &k1, const std::string &k2, float def)
{
    float v;
    const MetaValue *a = meta_of(m, k1);
    if (a)
        return as_f32(a, &v) ? v : def;
    return as_f32(meta_of(m, k2), &v) ? v : def;
}

std::string architecture(const Model &m)
{
    const MetaValue *v = meta_of(m, "general.architecture");
    return v && v->type == V_STR ? v->s : std::string("unknown");
}

int copy_str(const std::string &s, char *buf, size_t cap)
{
    if (!buf || cap <= s.size())
        return realm_set_error(REALM_INVALID_ARGUMENT,
                               "buffer of " + std::to_string(cap) + " bytes holds less than " +
                                   std::to_string(s.size() + 1));
    std::memcpy(buf, s.data(), s.size());
    buf[s.size()] = 0;
    return REALM_OK;
}

} // namespace

#define REALM_API extern "C" __attribute__((visibility("default")))

REALM_API int realm_hip_gguf_parse(const void *bytes, size_t len, uint64_t *model)
{
    if ((!bytes && len) || !model)
        return realm_set_error(REALM_INVALID_ARGUMENT, "gguf_parse needs bytes and a handle slot");
    Model m;
    GG_TRY(parse(static_cast<const uint8_t *>(bytes), len, &m));
    std::lock_guard<std::mutex> lk(g_gguf_mu);
    *model = g_next_model++;
    g_models.emplace(*model, std::move(m));
    return REALM_OK;
}

REALM_API int realm_hip_gguf_info(uint64_t model, uint32_t *version, uint64_t *tensor_count,
                                  uint64_t *kv_count, uint64_t *data_offset)
{
    std::lock_guard<std::mutex> lk(g_gguf_mu);
    Model *m;
    GG_TRY(get_model(model, &m));
    if (version)
        *version = m->version;
    if (tensor_count)
        *tensor_count = m->tensor_count;
    if (kv_count)
        *kv_count = m->kv_count;
    if (data_offset)
        *data_offset = m->data_offset;
    return REALM_OK;
}

REALM_API int realm_hip_gguf_tensor(uint64_t model, size_t index, char *name, size_t name_cap,
                                    int *ggml_type, uint32_t *n_dims, uint64_t *dims4,
                                    uint64_t *abs_offset, uint64_t *nbytes)
{
    std::lock_guard<std::mutex> lk(g_gguf_mu);
    Model *m;
    GG_TRY(get_model(model, &m));
    if (index >= m->tensors.size())
        return realm_set_error(REALM_INVALID_ARGUMENT, "tensor index " + std::to_string(index) +
                                                           " out of range");
    const Tensor &t = m->tensors[index];
    if (name)
        GG_TRY(copy_str(t.name, name, name_cap));
    if (ggml_type)
        *ggml_type = t.type;
    if (n_dims)
        *n_dims = (uint32_t)t.dims.size();
    if (dims4)
        for (size_t d = 0; d < 4; ++d)
            dims4[d] = d < t.dims.size() ? t.dims[d] : 1;
    if (abs_offset)
        *abs_offset = t.abs;
    if (nbytes)
        *nbytes = t.nbytes;
    return REALM_OK;
}

REALM_API int realm_hip_gguf_find(uint64_t model, const char *name, size_t *index)
{
    if (!name || !index)
        return realm_set_error(REALM_INVALID_ARGUMENT, "gguf_find needs a name and an index slot");
    std::lock_guard<std::mutex> lk(g_gguf_mu);
    Model *m;
    GG_TRY(get_model(model, &m));
    auto it = m->by_name.find(name);
    if (it == m->by_name.end())
        return realm_set_error(REALM_INVALID_ARGUMENT, std::string("no tensor named ") + name);
    *index = it->second;
    return REALM_OK;
}

REALM_API int realm_hip_gguf_meta_u32(uint64_t model, const char *key, uint32_t *out)
{
    if (!key || !out)
        return realm_set_error(REALM_INVALID_ARGUMENT, "gguf_meta_u32 needs a key and a slot");
    std::lock_guard<std::mutex> lk(g_gguf_mu);
    Model *m;
    GG_TRY(get_model(model, &m));
    if (!as_u32(meta_of(*m, key), out))
        return realm_set_error(REALM_INVALID_ARGUMENT, std::string("no integer metadata ") + key);
    return REALM_OK;
}

REALM_API int realm_hip_gguf_meta_str(uint64_t model, const char *key, char *buf, size_t cap)
{
    if (!key)
        return realm_set_error(REALM_INVALID_ARGUMENT, "gguf_meta_str needs a key");
    std::lock_guard<std::mutex> lk(g_gguf_mu);
    Model *m;
    GG_TRY(get_model(model, &m));
    const MetaValue *v = meta_of(*m, key);
    if (!v || v->type != V_STR)
        return realm_set_error(REALM_INVALID_ARGUMENT, std::string("no string metadata ") + key);
    return copy_str(v->s, buf, cap);
}

REALM_API int realm_hip_gguf_config(uint64_t model, realm_gguf_config *cfg)
{
    if (!cfg)
        return realm_set_error(REALM_INVALID_ARGUMENT, "gguf_config needs a config slot");
    std::lock_guard<std::mutex> lk(g_gguf_mu);
    Model *m;
    GG_TRY(get_model(model, &m));
    const std::string a = architecture(*m);
    cfg->vocab_size = cfg_u32(*m, a + ".vocab_size", "vocab_size", 32000);
    cfg->hidden_size = cfg_u32(*m, a + ".embedding_length", a + ".hidden_size", 2048);
    cfg->num_layers = cfg_u32(*m, a + ".block_count", a + ".num_layers", 22);
    cfg->num_heads = cfg_u32(*m, a + ".attention.head_count", a + ".num_heads", 32);
    cfg->num_kv_heads = cfg_u32(*m, a + ".attention.head_count_kv", a + ".num_kv_heads", 4);
    cfg->intermediate_size = cfg_u32(*m, a + ".feed_forward_length", a + ".intermediate_size", 5632);
    cfg->max_seq_len = cfg_u32(*m, a + ".context_length", a + ".max_seq_len", 2048);
    cfg->rms_norm_eps = cfg_f32(*m, a + ".attention.layer_norm_rms_epsilon", "rms_norm_eps", 1e-5f);
    cfg->rope_theta = cfg_f32(*m, a + ".rope.freq_base", "rope_theta", 10000.0f);
    return REALM_OK;
}

REALM_API int realm_hip_gguf_register(uint64_t model, const void *bytes, size_t len,
                                      size_t *registered)
{
    if (!bytes)
        return realm_set_error(REALM_INVALID_ARGUMENT, "gguf_register needs the image bytes");
    // the tensors to upload, read under the lock; registration itself runs
    // without it (it takes the library's own locks)
    std::vector<std::pair<size_t, Tensor>> todo;
    {
        std::lock_guard<std::mutex> lk(g_gguf_mu);
        Model *m;
        GG_TRY(get_model(model, &m));
        for (size_t i = 0; i < m->tensors.size(); ++i) {
            const Tensor &t = m->tensors[i];
            const bool quant = t.type == REALM_GGML_Q4_K || t.type == REALM_GGML_Q6_K ||
                               t.type == REALM_GGML_Q8_0 || t.type == REALM_GGML_Q4_0 ||
                               t.type == REALM_GGML_Q4_1 || t.type == REALM_GGML_Q5_0 ||
                               t.type == REALM_GGML_Q5_1 || t.type == REALM_GGML_Q8_1;
            if (!quant || t.dims.size() != 2 || t.weight)
                continue;
            if (t.abs > len || t.nbytes > len - t.abs)
                return realm_set_error(REALM_MODEL_PARSE_ERROR,
                                       "tensor " + t.name + " extends past the end of the image");
            todo.emplace_back(i, t);
        }
    }
    // the device footprint of all of them first (the reference's Q2_K / Q3_K
    // / Q5_K / Q8_K stay resident dequantized, 4 bytes per weight; the
    // 32-element formats take the q8m layout, 1.125 bytes per weight plus
    // padding): an image that cannot fit is refused before anything is
    // registered
    size_t need = 0, free_bytes = 0;
    for (auto &it : todo) {
        const Tensor &t = it.second;
        const size_t elems = (size_t)(t.dims[0] * t.dims[1]);
        const bool kq = t.type == REALM_GGML_Q2_K || t.type == REALM_GGML_Q3_K ||
                        t.type == REALM_GGML_Q5_K || t.type == REALM_GGML_Q8_K;
        const bool q8m = t.type == REALM_GGML_Q4_0 || t.type == REALM_GGML_Q4_1 ||
                         t.type == REALM_GGML_Q5_0 || t.type == REALM_GGML_Q5_1 ||
                         t.type == REALM_GGML_Q8_1;
        need += kq ? elems * 4 : q8m ? elems + elems / 8 + 4096 : (size_t)t.nbytes + (size_t)t.nbytes / 8;
    }
    GG_TRY(realm_device_free_bytes(&free_bytes));
    if (need > free_bytes)
        return realm_set_error(REALM_OUT_OF_MEMORY,
                               "registering the image's quantized tensors needs about " +
                                   std::to_string(need) + " bytes of device memory, " +
                                   std::to_string(free_bytes) + " are free");
    size_t count = 0;
    for (auto &it : todo) {
        const Tensor &t = it.second;
        // ggml order: dims[0] is the row length K, dims[1] the row count N
        uint64_t h = 0;
        GG_TRY(realm_hip_weights_register(t.type, static_cast<const uint8_t *>(bytes) + t.abs,
                                          (size_t)t.nbytes, (size_t)t.dims[1], (size_t)t.dims[0],
                                          &h));
        std::lock_guard<std::mutex> lk(g_gguf_mu);
        Model *m;
        if (get_model(model, &m) != REALM_OK) { // released meanwhile
            realm_hip_weights_release(h);
            return realm_set_error(REALM_INVALID_ARGUMENT, "GGUF model released during registration");
        }
        m->tensors[it.first].weight = h;
        ++count;
    }
    if (registered)
        *registered = count;
    return REALM_OK;
}

REALM_API int realm_hip_gguf_weight(uint64_t model, const char *name, uint64_t *weight,
                                    size_t *n, size_t *k)
{
    if (!name || !weight)
        return realm_set_error(REALM_INVALID_ARGUMENT, "gguf_weight needs a name and a slot");
    std::lock_guard<std::mutex> lk(g_gguf_mu);
    Model *m;
    GG_TRY(get_model(model, &m));
    auto it = m->by_name.find(name);
    if (it == m->by_name.end())
        return realm_set_error(REALM_INVALID_ARGUMENT, std::string("no tensor named ") + name);
    const Tensor &t = m->tensors[it->second];
    if (!t.weight)
        return realm_set_error(REALM_BACKEND_UNSUPPORTED,
                               std::string("tensor ") + name + " is not a registered weight");
    *weight = t.weight;
    if (n)
        *n = (size_t)t.dims[1];
    if (k)
        *k = (size_t)t.dims[0];
    return REALM_OK;
}

REALM_API int realm_hip_gguf_release(uint64_t model)
{
    std::vector<uint64_t> weights;
    {
        std::lock_guard<std::mutex> lk(g_gguf_mu);
        auto it = g_models.find(model);
        if (it == g_models.end())
            return realm_set_error(REALM_INVALID_ARGUMENT,
                                   "unknown GGUF model handle " + std::to_string(model));
        for (const Tensor &t : it->second.tensors)
            if (t.weight)
                weights.push_back(t.weight);
        g_models.erase(it);
    }
    int rc = REALM_OK;
    for (uint64_t h : weights)
        if (int r = realm_hip_weights_release(h))
            rc = r;
    return rc;
}
